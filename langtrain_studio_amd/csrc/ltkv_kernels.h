// Internal launcher interface between the host block manager (ltkv_cache.cpp)
// and the gfx950 kernels (ltkv_kernels.hip). Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>

namespace ltkv {

constexpr int kBlock = 16;  // tokens per block (kv.rs:13)

// Geometry of one layer of a pool: element (block, slot, head, i) lives at
// block*block_stride + head*head_stride + slot*slot_stride + i.
struct PoolGeom {
  int64_t n_blocks;
  int64_t block_stride;  // elements per block (16 * kv_dim)
  int64_t slot_stride;   // elements between consecutive slots of a block
  int64_t head_stride;   // elements between consecutive kv heads of a block
  int kv_dim;
  int elem;              // bytes per element: 1 (q8_0 quants), 2 (f16) or 4 (f32)
};

// Kernel 1 for q8_0 cells (elem 1): quants into k/v_layer, per-32 f16 scales
// into k/v_scale ([cell][kv_dim / 32]).
// With order (n entries), launch row i is source row order[i]; entries outside
// [0, n_rows) are skipped.
hipError_t launch_write_q8(const PoolGeom &g, void *k_layer, void *v_layer, void *k_scale,
                           void *v_scale, const int32_t *slots, const float *k, const float *v,
                           int64_t n, int64_t src_stride, hipStream_t s, const int32_t *order = nullptr,
                           int64_t n_rows = 0);

hipError_t launch_write(const PoolGeom &g, void *k_layer, void *v_layer, const int32_t *slots,
                        const float *k, const float *v, int64_t n, int64_t src_stride,
                        hipStream_t s, const int32_t *order = nullptr, int64_t n_rows = 0);

// RoPE geometry: table [max_pos][rope_dim / 2] of (cos, sin) of pos * inv_freq[i].
struct RopeGeom {
  const float *table;
  int max_pos, rope_dim, head_dim, neox;
};

// Kernel 1 with RoPE: K rotated into the pool, V appended, Q (optional,
// [n][q_stride] with n_heads heads) rotated in place.
hipError_t launch_write_rope(const PoolGeom &g, void *k_layer, void *v_layer, const int32_t *slots,
                            const int32_t *positions, const float *k, const float *v, float *q,
                            int64_t n, int64_t src_stride, int64_t q_stride, int n_heads,
                            const RopeGeom &r, hipStream_t s);

// The same for q8_0 cells: K rotated then quantised per 32 elements, V
// quantised, Q rotated in place.
hipError_t launch_write_rope_q8(const PoolGeom &g, void *k_layer, void *v_layer, void *k_scale, void *v_scale,
                               const int32_t *slots, const int32_t *positions, const float *k, const float *v,
                               float *q, int64_t n, int64_t src_stride, int64_t q_stride, int n_heads,
                               const RopeGeom &r, hipStream_t s);

// Kernel 2 over (src, dst) block pairs of every layer; `bulk` selects the
// form for large batches (pairs in destination order, see launch_copy_order).
// Most pairs one launch_copy_blocks call takes for this pool geometry.
int64_t copy_max_pairs(const PoolGeom &g, int n_layers, bool bulk);
hipError_t launch_copy_blocks(const PoolGeom &g, int n_layers, void *k_pool, void *v_pool,
                              const int32_t *pairs, int64_t n_pairs, bool bulk, hipStream_t s);

// Copy pairs bucketed by destination block (2^6 blocks a bucket), ascending:
// `counts` holds copy_order_buckets(n_blocks) int32 that are zero on entry
// and zero again on exit; `cursors` as many; `sorted` 2 n_pairs int32.
int64_t copy_order_buckets(int64_t n_blocks);
hipError_t launch_copy_order(const int32_t *pairs, int64_t n_pairs, int64_t n_blocks, int32_t *counts,
                             int32_t *cursors, int32_t *sorted, hipStream_t s);

// Table entries outside the pool are not copied and set kFaultTable in
// status[0] (see AttnArgs::status).
hipError_t launch_gather(const PoolGeom &g, const void *k_layer, const void *v_layer,
                         const int32_t *tables, int64_t table_stride, const int32_t *lens,
                         const int64_t *out_offsets, int64_t n, void *k_out, void *v_out,
                         int32_t *status, hipStream_t s);

// Fault word int32[4]: moves words 0..1 (fault bits, query) into words 2..3
// and clears them, in stream order.
hipError_t launch_status_take(int32_t *status, hipStream_t s);
// Resident block tables: updates (row, col, value) triples (col -1: the
// row's length in blocks), and the slot mapping of (row, position) tokens.
// Up to kTableUpdateArgs triples passed by value (kernel arguments hold 4 KB).
constexpr int kTableUpdateArgs = 320;
struct TableUpdates {
  int32_t n;
  int32_t t[3 * kTableUpdateArgs];
};
hipError_t launch_table_update_args(int32_t *tables, int32_t *counts, int64_t width, int64_t n_rows,
                                    const TableUpdates &u, hipStream_t s);
hipError_t launch_table_update(int32_t *tables, int32_t *counts, int64_t width, int64_t n_rows,
                               const int32_t *upd, int64_t n, hipStream_t s);
hipError_t launch_slot_mapping(const int32_t *tables, const int32_t *counts, int64_t width,
                               int64_t n_rows, const int32_t *rows, const int64_t *pos, int64_t n,
                               int32_t *out, hipStream_t s);

struct AttnArgs {
  const void *k_layer, *v_layer;
  const void *k_scale, *v_scale;  // q8_0 pools: per-32 f16 scales of the layer, else null
  const float *q;
  const int32_t *tables;
  int64_t table_stride;
  const int32_t *lens;
  float *out;
  float *part_o;   // [n][n_heads][max_parts][head_dim] partial numerators
  float *part_ml;  // [n][n_heads][max_parts][2] partial (max, sum), log2 domain
  int64_t n;
  int n_heads, n_kv_heads, head_dim;
  float scale;
  int part_tokens, max_parts;  // part_tokens 0 or kPartCap: per-query partition_tokens(len, part_tokens)
  // The matrix-core decode kernel cuts each partition into `split`
  // (partition_tokens(len) / split tokens each, split 1 or 2); max_parts
  // counts the finer partitions. attention_split gives it for a shape.
  int split;
  // Resident block tables: query i reads row rows[i] of `tables` (rows ==
  // nullptr: row i); rows outside [0, n_rows) read row 0.
  const int32_t *rows;
  int64_t n_rows;
  // Lengths are cut to max_len tokens (at most table_stride * 16); the grid's
  // max_parts covers max_len.
  int64_t max_len;
  // Compute units of the device (the matrix-core decode kernel's wave slots;
  // 0: no runs of partitions per wave).
  int cu_count;
  // The caller knows no query needs the merge pass: every query has one
  // partition, and none with group partials has an empty remainder (the
  // matrix-core kernel folds group partials of single-partition queries).
  bool merge_free;
  // The caller knows the context kernel has nothing to do: every query has
  // group partials and an empty remainder, so only the merge runs (it folds
  // the group partials by itself).
  bool pass_empty;
  // Fused append (f16 pools, matrix-core kernel): query i's new K/V row
  // (new_k/new_v row i, f32, row stride new_stride) is written to cell
  // new_slots[i], which must be position lens[i] - 1 of the query's table,
  // and attended from registers. nullptr: no fused append.
  const int32_t *new_slots;
  const float *new_k, *new_v;
  int64_t new_stride;
  // Group partials folded into each query's result (planned attention), or
  // pre_parts == nullptr: query i has pre_parts[i] partials at pre_o/pre_ml
  // slot (i * n_heads + head) * max_pre_parts + p; -1: its group wrote the
  // output and nothing else reads its context.
  const int32_t *pre_parts;
  const float *pre_o, *pre_ml;
  int max_pre_parts;
  // Queries the launch covers: qmap[0..n) (query indices), or all n when null.
  const int32_t *qmap;
  // f16 pools: the vector-ALU kernels (attn16_kernel / attn_kernel) instead
  // of the matrix-core one (LTKV_ENGINE_VALU); they write partials for every
  // multi-partition query and leave group partials to the merge.
  bool valu;
  // Fault word (int32[2], or nullptr): a table entry outside the pool that a
  // query's context covers (read as block 0) ORs 1 into status[0], a fused
  // append whose cell is not position lens[i] - 1 of the query's table ORs
  // 2; status[1] gets the query. Kernels only ever set bits.
  int32_t *status;
};

// Partition policy kPartCap (part_tokens -1): 1024-token partitions (the
// last one the rest) for queries over 2048 tokens, four equal ones below.
constexpr int kPartCap = -1;

// Context tokens per attention partition when none is fixed (part_tokens 0):
// four partitions of a query up to 4096 tokens (at least 64 tokens each),
// 1024 tokens beyond; with kPartCap already beyond 2048 tokens. Either way it
// depends on the query's own length only, so a query's result never depends
// on the rest of the batch.
__host__ __device__ inline int partition_tokens(int64_t len, int fixed) {
  if (fixed > 0) return fixed;
  if (len > (fixed == kPartCap ? 2048 : 4096)) return 1024;
  const int64_t p = ((len + 3) / 4 + 63) / 64 * 64;
  return p < 64 ? 64 : (int)p;
}

// ceil(len / pt) for 0 <= len < 2^31 and pt > 0, in 32-bit arithmetic (a
// 64-bit division is a long instruction sequence on the vector ALU, on the
// path from a wave's start to its first loads).
__host__ __device__ inline int div_up_tokens(int64_t len, int pt) {
  return (int)(((uint32_t)len + (uint32_t)pt - 1u) / (uint32_t)pt);
}

// A query's partition size with the matrix-core kernel's cut (split 1 or 2).
__host__ __device__ inline int split_partition(int64_t len, int part_tokens, int split) {
  const int pt = partition_tokens(len, part_tokens);
  return split == 1 ? pt : (split == 2 ? pt >> 1 : pt / split);
}

// Upper bound of partitions per query for contexts up to max_tokens (the
// same for both per-query policies: at most four up to 4096 tokens).
inline int max_partitions(int64_t max_tokens, int fixed) {
  if (fixed > 0) return (int)((max_tokens + fixed - 1) / fixed);
  const int64_t beyond = (max_tokens + 1023) / 1024;
  return (int)(beyond > 4 ? beyond : 4);
}

// Workspace of launch_decode_attention: partition partials (bytes == 0 when
// one partition covers every query).
struct AttnWorkspace {
  int64_t part_o_off, part_ml_off, bytes;
};
// always: partials even when one partition covers every query (the planned
// path merges them with shared-prefix partials).
AttnWorkspace attention_workspace(int64_t n, int n_heads, int head_dim, int max_parts,
                                  bool always = false);
// Shapes of the tuned decode kernels (head_dim 64 or 128, group 1..8) and of
// every kernel (any group, head_dim up to 1024: the generic kernel, one
// work-group per query head, no partitions, no group partials).
bool attention_tuned(int elem, int head_dim, int group);
bool attention_supported(int elem, int head_dim, int group);
// Decode kernels on f16 and q8_0 pools read two adjacent kv heads per wave
// when the group has at most 4 query heads and the kv heads pair up (the
// wave's 2 x group query heads fill the 16 columns of its products). The
// partition divisor (1 or 2) of such a shape, 1 otherwise. It never depends
// on the batch: a query's result bits depend on its own inputs only.
int attention_split(int elem, int group, int n_kv_heads);
// The per-query partition policy of a shape (and engine: valu for
// LTKV_ENGINE_VALU) when none is fixed: kPartCap or 0.
int attention_part_policy(int elem, int group, int n_kv_heads, bool valu);
hipError_t launch_decode_attention(const PoolGeom &g, const AttnArgs &a, hipStream_t s);

// One work-group of shared-prefix attention (mq_attn_kernel): the query rows
// of n_members members of a prefix-sharing group (every query head of kv
// head kvh) against tokens [t0, t1) of the group's shared blocks.
struct MqJob {
  int32_t table;               // offset of the group's block table in the tables array
  int32_t t0, t1;              // token range
  int32_t member0, n_members;  // members[2*member0 ...]: (query, token limit) pairs
  int32_t part;                // partial slot of this token range
  int32_t kvh;
  int32_t direct;              // 1: the rows' only contribution; write the output
};
int mq_rows(int elem, int head_dim);  // query rows per work-group
constexpr int kMqMaxRange = 16384;  // longest token range of one group job (its block ids sit in LDS)

struct MqArgs {
  const void *k_layer, *v_layer;
  const float *q;
  const int32_t *tables;
  const MqJob *jobs;
  int n_jobs;
  const int32_t *members;
  const void *k_scale, *v_scale;  // q8_0 scale pools of the layer (nullptr for f16)
  float *pre_o, *pre_ml;  // partial slots, laid out as AttnArgs::pre_o/pre_ml
  float *out;             // outputs of direct jobs
  int n_heads, n_kv_heads, head_dim;
  float scale;
  int max_pre_parts;
  // Products with Q and P rounded to f16 (LTKV_PLAN_F16_PRODUCTS), else
  // with f16 hi + lo pairs (f32 accuracy).
  bool f16_products;
};
bool mq_supported(int elem, int head_dim, int group);
hipError_t launch_mq_attention(const PoolGeom &g, const MqArgs &a, hipStream_t s);

// Scratch of the allocation-free decode attention: a static device array of
// kScratchBytes on every device the library runs on. scratch_address gives
// its address on `device`, which must be the current device on the first
// call for that device (looked up once per device with hipGetSymbolAddress,
// then kept).
constexpr size_t kScratchBytes = size_t{32} << 20;
constexpr int kMaxScratchDevices = 64;
hipError_t scratch_address(int device, void **ptr);

}  // namespace ltkv
