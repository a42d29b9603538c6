/*
 * ltkv.h - C ABI of the MI355X-native paged KV cache.
 *
 * Drop-in for the Langtrain engine's paged KV-cache path. The reference is
 * Rust: the cache type langtrain_native::kv::KvCache
 * (engine/crates/native/src/kv.rs:15-188) and its callers, the KV segment of
 * Model::forward (engine/crates/native/src/model.rs:380-475) and
 * NativeBackend::decode / kv_remove / kv_copy
 * (engine/crates/native/src/lib.rs:163-198, behind the Backend trait of
 * engine/crates/engine/src/backend.rs:17-45). Each entry point below names
 * the reference item it replaces.
 *
 * Model:
 *  - Host metadata (block allocator, block tables, refcounts) lives in the
 *    library and has the exact semantics of kv.rs: 16-token blocks, a LIFO
 *    free stack handing out blocks 0,1,2,... on a fresh cache, refcounted
 *    prefix sharing and copy-on-write on the first write into a shared block.
 *  - K and V pools live in device memory (HBM) and are owned by the cache.
 *    Layout: [layer][block][slot][kv_dim] per pool, as kv.rs:20-22.
 *  - Device work is enqueued, in call order, on the cache's stream
 *    (ltkv_set_stream; default: the null stream of the cache's device).
 *    Device pointers passed in must be valid on that stream.
 *  - One thread mutates a cache at a time, like KvCache's &mut self methods.
 *
 * Status codes: every int-returning call returns LTKV_OK or an LTKV_ERR_*
 * code and sets a thread-local message readable with ltkv_last_error(). The
 * messages of the two reference errors are reproduced verbatim:
 *   LTKV_ERR_FULL       "KV cache full"                               (kv.rs:71)
 *   LTKV_ERR_NONCONTIG  "seq S: position P is not contiguous (length L)" (kv.rs:88-91)
 */
#ifndef LTKV_H
#define LTKV_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__)
#define LTKV_API __attribute__((visibility("default")))
#else
#define LTKV_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define LTKV_BLOCK 16 /* tokens per block: kv.rs:13 `pub const BLOCK: usize = 16` */

typedef struct ltkv_cache ltkv_cache;

enum {
  LTKV_OK = 0,
  LTKV_ERR_FULL = 1,      /* allocator exhausted (kv.rs:67-74) */
  LTKV_ERR_NONCONTIG = 2, /* append at pos != len (kv.rs:87-92) */
  LTKV_ERR_RANGE = 3,     /* index out of range (the reference panics: kv.rs:147) */
  LTKV_ERR_HIP = 4,       /* a HIP runtime call or kernel launch failed */
  LTKV_ERR_ARG = 5        /* invalid argument */
};

/* ltkv_create device argument for a metadata-only cache: allocator, tables
 * and refcounts with no device pools. Every device op on it fails with
 * LTKV_ERR_ARG (there is no host compute path). */
#define LTKV_NO_DEVICE (-1)

/* Storage element type. F16 is the reference's (kv.rs:5-6); F32 stores the
 * f32 input unrounded (same algorithm without the rounding step). Q8_0
 * stores each 32-element run of a row as 32 int8 quants plus an f16 scale d
 * (the Q8_0 block of quant.rs:188-193, quantised as quant.rs:785-791 and
 * read back as d * q): quants in the K/V pools ([n_blocks][16][kv_dim]
 * bytes), scales in K/V scale pools ([n_blocks][kv_dim/32][16] f16: per
 * block, the 16 slots of each 32-element group are adjacent, so one kv
 * head's scales of a block are one contiguous run).
 * kv_dim must be a multiple of 32 (head_dim too for the RoPE append). Gather
 * and rows have no Q8_0 form (LTKV_ERR_ARG). */
enum { LTKV_F16 = 0, LTKV_F32 = 1, LTKV_Q8_0 = 2 };

/* Thread-local message of the last failing call on this thread. */
LTKV_API const char *ltkv_last_error(void);

/* ---- lifecycle ---------------------------------------------------------- */

/* KvCache::new(n_layers, kv_dim, n_tokens) (kv.rs:35-48): ceil(n_tokens/16)
 * blocks, zero-filled K and V pools on HIP device `device` (or none for
 * LTKV_NO_DEVICE), free stack (0..n_blocks).rev(). Any kv_dim >= 1 (Q8_0:
 * a multiple of 32); rows whose byte length is a multiple of 16 take the
 * vectorised kernels, others element-wise ones. */
LTKV_API int ltkv_create(size_t n_layers, size_t kv_dim, size_t n_tokens, int dtype, int device,
                ltkv_cache **out);
LTKV_API void ltkv_destroy(ltkv_cache *c);

/* Stream on which all device work of this cache is enqueued (hipStream_t). */
LTKV_API int ltkv_set_stream(ltkv_cache *c, void *hip_stream);

/* ---- queries (kv.rs:50-60,185-187) ------------------------------------- */

LTKV_API size_t ltkv_capacity(const ltkv_cache *c);    /* KvCache::capacity: n_blocks*16 */
LTKV_API size_t ltkv_bytes(const ltkv_cache *c);       /* KvCache::bytes: K+V pool (and scale pool) bytes */
LTKV_API size_t ltkv_len(const ltkv_cache *c, uint32_t seq); /* KvCache::len (0 if unknown) */
LTKV_API size_t ltkv_free_blocks(const ltkv_cache *c); /* KvCache::free_blocks */
LTKV_API size_t ltkv_n_blocks(const ltkv_cache *c);
LTKV_API size_t ltkv_kv_dim(const ltkv_cache *c);      /* KvCache::kv_dim */
LTKV_API uint32_t ltkv_refcount(const ltkv_cache *c, uint32_t block); /* refs[block]; 0 if out of range */
LTKV_API uint64_t ltkv_cow_copies(const ltkv_cache *c); /* copy-on-write block copies made so far */

/* ---- block management (host; copy-on-write copies go to the stream) ----- */

/* KvCache::append(seq, pos) (kv.rs:85-121): reserve the cell for pos (must
 * equal len(seq)); returns (block, slot). A copy-on-write of the sequence's
 * shared last block is enqueued on the stream before returning. */
LTKV_API int ltkv_append(ltkv_cache *c, uint32_t seq, size_t pos, uint32_t *block, uint32_t *slot);

/* The cell claim of Model::forward (model.rs:380-383) for a whole batch:
 * append(seqs[i], pos[i]) in order, writing slot_mapping[i] = block*16+slot
 * (host array). All copy-on-write copies of the batch are enqueued as one
 * launch before returning, so they precede any later write. On error the
 * claims before the failing entry stay made (as collect::<Result<_>>()),
 * their copies are still enqueued, and *n_done (optional) says how many. */
LTKV_API int ltkv_append_batch(ltkv_cache *c, size_t n, const uint32_t *seqs, const uint64_t *pos,
                      int32_t *slot_mapping, size_t *n_done);

/* KvCache::truncate(seq, from) (kv.rs:153-169): keep ceil(from/16) blocks;
 * from == 0 drops the sequence; unknown seq is a no-op. Backend::kv_remove. */
LTKV_API void ltkv_truncate(ltkv_cache *c, uint32_t seq, size_t from);

/* KvCache::share(src, dst, len) (kv.rs:172-183): dst becomes the first
 * min(len, len(src)) tokens of src, sharing blocks. Backend::kv_copy. */
LTKV_API void ltkv_share(ltkv_cache *c, uint32_t src, uint32_t dst, size_t len);

/* Block table of seq (the Seq::blocks of kv.rs:28-32). Writes up to cap
 * entries; *n_blocks gets the table length. LTKV_ERR_RANGE if cap is short. */
LTKV_API int ltkv_block_table(const ltkv_cache *c, uint32_t seq, int32_t *out, size_t cap, size_t *n_blocks);

/* Row-major [n][stride] tables for n sequences (host array), for the device
 * ops below; entries past a table's end are set to -1. */
LTKV_API int ltkv_block_tables(const ltkv_cache *c, size_t n, const uint32_t *seqs, int32_t *out,
                      size_t stride);

/* Seed the free stack of a fresh cache (no sequences) so that successive
 * allocations return order[0], order[1], ...; order is a permutation of
 * 0..n_blocks-1. The reference's own order is 0,1,2,... (kv.rs:45). */
LTKV_API int ltkv_init_free_order(ltkv_cache *c, const uint32_t *order, size_t n);

/* ---- device ops (enqueued on the cache's stream) ----------------------- */

/* Kernel 1, slot-mapped append: KvCache::write (kv.rs:123-131) for n rows,
 * as the per-token loop of model.rs:414-429. Row i of d_k/d_v (f32, row
 * stride src_stride >= kv_dim elements) goes to cell d_slot_mapping[i] =
 * block*16+slot of `layer`, rounded f32->f16 RNE (F16), stored as is
 * (F32) or quantised per 32 elements (Q8_0: amax = max |x| ignoring NaN,
 * d = amax / 127, q = round-half-away(x / d) saturated to int8, NaN -> 0,
 * d stored as f16 RNE). Negative or out-of-range slots are skipped. */
LTKV_API int ltkv_write(ltkv_cache *c, size_t layer, size_t n, const int32_t *d_slot_mapping,
               const float *d_k, const float *d_v, size_t src_stride);

/* Host only: the rows of a claimed batch (slot_mapping[0..n), host memory, as
 * ltkv_append_batch returned it) grouped by block in ascending block order,
 * rows of one block in batch order (a block's rows in a claim are one
 * sequence's increasing positions, kv.rs:85-121, so in increasing slot
 * order): order[0..*m) receives the row indices; skipped cells (negative or
 * past the pool) are left out. A counting sort over the cache's blocks, or a
 * sort of the rows when they are few against the pool. No counterpart in the
 * reference (its write loop, model.rs:414-429, takes tokens in batch order):
 * bulk appends written in this order (ltkv_write_ordered) store into the
 * pool in ascending address order, which HBM takes faster than the scattered
 * order of a fragmented pool. */
LTKV_API int ltkv_cell_order(const ltkv_cache *c, size_t n, const int32_t *slot_mapping, int32_t *order,
                    size_t *m);

/* ltkv_write over the m rows d_order[0..m) (device memory) of a batch of n
 * rows: row d_order[j] of d_k / d_v goes to cell d_slot_mapping[d_order[j]];
 * entries outside [0, n) are skipped. The same cells and bits as ltkv_write
 * of the batch when d_order lists each row once (as ltkv_cell_order gives). */
LTKV_API int ltkv_write_ordered(ltkv_cache *c, size_t layer, size_t n, const int32_t *d_slot_mapping,
                       const float *d_k, const float *d_v, size_t src_stride, size_t m,
                       const int32_t *d_order);

/* RoPE of Model::rope (model.rs:291-308) with the table of model.rs:263-265:
 * inv_freq[i] = base^(-2i / rope_dim), angle = pos * inv_freq[i], cos/sin by
 * the host libm (as the reference), pairs (2i, 2i+1) or, with neox, (i, i +
 * rope_dim/2); dimensions past rope_dim are not rotated. Builds the
 * [max_positions][rope_dim/2] table in HBM for ltkv_write_rope. */
LTKV_API int ltkv_rope_init(ltkv_cache *c, float base, size_t rope_dim, size_t head_dim, int neox,
                   size_t max_positions);

/* model.rs:414-429 in one launch: RoPE on each token's K (then written into
 * its cell as ltkv_write does) and, when d_q is not null, on its Q rows
 * ([n][q_stride], n_heads heads) in place; V appended unrotated. Tokens with
 * a position outside the table are skipped (nothing written). Bit-identical
 * to the reference's f32 rotation (no fused multiply-add) and f16 rounding
 * (Q8_0 cells: the rotated K row quantised as ltkv_write does). */
LTKV_API int ltkv_write_rope(ltkv_cache *c, size_t layer, size_t n, const int32_t *d_slot_mapping,
                    const int32_t *d_positions, const float *d_k, const float *d_v, size_t src_stride,
                    float *d_q, size_t q_stride, size_t n_heads);

/* Kernel 2, block copy: the copy-on-write body of kv.rs:99-110 (all layers,
 * K and V) for n pairs d_pairs[2i] = src block, d_pairs[2i+1] = dst block.
 * ltkv_append and ltkv_append_batch launch it themselves; exposed for bulk
 * use. Pairs with an out-of-range block are skipped. One call takes at most
 * (2^32 - 1) / (n_layers * 2 * ceil(16 * kv_dim * elem / 16 KiB)) pairs
 * (4096 pairs and more; 8 KiB chunks below that) and INT32_MAX in any case,
 * e.g. 33 554 431 pairs for 32 layers of kv_dim 1024 f16; more is
 * LTKV_ERR_ARG. */
LTKV_API int ltkv_copy_blocks(ltkv_cache *c, size_t n, const int32_t *d_pairs);

/* Kernel 3, gather: KvCache::rows(layer, seq, len) collected (kv.rs:133-150)
 * for n sequences. Sequence i has table d_tables[i*table_stride ...] and
 * length d_lens[i] <= table_stride*16; its rows go to row d_out_offsets[i]
 * onward of d_k_out / d_v_out ([rows][kv_dim], cache dtype), bit-exact. A
 * table entry outside the pool copies nothing and is reported by
 * ltkv_synchronize (the reference panics, kv.rs:147). */
LTKV_API int ltkv_gather(ltkv_cache *c, size_t layer, size_t n, const int32_t *d_tables,
                size_t table_stride, const int32_t *d_lens, const int64_t *d_out_offsets,
                void *d_k_out, void *d_v_out);

/* Kernel 4, GQA paged decode attention: the attention closure of
 * model.rs:431-475 for n queries. Query i (d_q row i, [n_heads*head_dim] f32)
 * attends over positions 0..d_lens[i]-1 of the table at
 * d_tables[i*table_stride]; query head h uses kv head h/(n_heads/n_kv_heads).
 * Softmax of q.k*scale over the positions, times V; d_out is
 * [n][n_heads*head_dim] f32. Any group size and head_dim <= 1024: head_dim
 * 64 or 128 with groups of 1..8 take the tuned kernels, other shapes a
 * generic one (one work-group per query head, whole contexts).
 * d_lens[i] == 0 yields zeros. A table entry outside the pool is read as
 * block 0 and reported by ltkv_synchronize (the reference panics, kv.rs:147).
 * Q may have any finite magnitude, as the reference's f32 scores allow
 * (model.rs:450,455-461): the matrix-core kernels (f16 and Q8_0 pools) take
 * q * scale * log2(e) as f16 hi + lo operands, and a query head whose
 * elements reach 65504 (|q| ~ 5.1e5 at head_dim 128) enters the products
 * scaled by 2^-e, its scores multiplied by 2^e afterwards (both exact). */
LTKV_API int ltkv_decode_attention(ltkv_cache *c, size_t layer, size_t n, size_t n_heads, size_t head_dim,
                          float scale, const float *d_q, const int32_t *d_tables,
                          size_t table_stride, const int32_t *d_lens, float *d_out);

/* Bytes of the per-device static scratch of ltkv_decode_attention_noalloc. */
#define LTKV_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)

/* ltkv_decode_attention that allocates nothing: same arguments, same
 * kernels, same results bit for bit, but the partition partials go to a
 * static device array of LTKV_NOALLOC_SCRATCH_BYTES on each device (held
 * until the process ends) instead of the cache's workspace, which
 * ltkv_decode_attention grows with hipMalloc on demand. A launch whose
 * partials need more fails with LTKV_ERR_ARG before anything is enqueued:
 * they take n * n_heads * P * (head_dim + 2) * 4 bytes, P counted for the
 * longest context the tables hold (T = table_stride * 16 tokens): 4 up to
 * 4096 tokens, ceil(T / 1024) beyond (or ceil(T / the size fixed with
 * ltkv_set_attention_partition)), doubled on Q8_0 pools whose kv heads
 * pair up with at most 4 query heads each. Every
 * call on a device shares that device's scratch: calls that overlap on one
 * device (other streams, other threads, caches on the same device) race.
 * No counterpart in the reference: for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). */
LTKV_API int ltkv_decode_attention_noalloc(ltkv_cache *c, size_t layer, size_t n, size_t n_heads,
                                           size_t head_dim, float scale, const float *d_q,
                                           const int32_t *d_tables, size_t table_stride,
                                           const int32_t *d_lens, float *d_out);

/* A decode step's append and attention in one launch: KvCache::write of
 * row i of d_k/d_v (f32, row stride src_stride) into cell d_slot_mapping[i]
 * (kv.rs:123-131), then ltkv_decode_attention over the same tables and
 * lengths (model.rs:414-475 for one layer). The cell must be position
 * d_lens[i] - 1 of query i's table (the cell the step's claim returned for
 * that query) and no two queries may read one sequence's new cells (one new
 * token per sequence, as in a decode step); then results and pools are
 * bit-identical to ltkv_write followed by ltkv_decode_attention (a cell that
 * is not position d_lens[i] - 1 is reported by ltkv_synchronize as
 * LTKV_ERR_ARG). A negative or out-of-range cell is skipped, as by
 * ltkv_write. On f16 pools the
 * attention kernel writes and uses each new row itself; on f32 and Q8_0
 * pools, and on f16 pools set to LTKV_ENGINE_VALU, this is ltkv_write
 * followed by ltkv_decode_attention. No reference counterpart: the reference
 * writes then attends per layer. */
LTKV_API int ltkv_append_decode_attention(ltkv_cache *c, size_t layer, size_t n, size_t n_heads,
                                          size_t head_dim, float scale, const float *d_q,
                                          const int32_t *d_tables, size_t table_stride,
                                          const int32_t *d_lens, const int32_t *d_slot_mapping,
                                          const float *d_k, const float *d_v, size_t src_stride,
                                          float *d_out);

/* Tokens per context partition of the decode attention split (multiple of
 * 64), or 0 (the default) for the per-query policy: a query is split into
 * four partitions of ceil(len/4) rounded up to 64 tokens (at least 64) up to
 * 4096 tokens, and into 1024-token partitions beyond; on f16 pools (the
 * matrix-core engine) the 1024-token partitions start beyond 2048 tokens.
 * Either way a query's result depends only on its own inputs, the cache's
 * shape and its engine, never on the rest of the batch. Tuning knob. */
LTKV_API int ltkv_set_attention_partition(ltkv_cache *c, size_t tokens);

/* Engines of the decode attention kernels (ltkv_set_attention_engine). */
#define LTKV_ENGINE_AUTO 0 /* f16 and Q8_0 pools on the matrix cores, f32 on the vector ALU */
#define LTKV_ENGINE_VALU 1 /* f16 pools on the vector ALU as well */

/* Which kernels run decode attention (ltkv_decode_attention, _rows, _noalloc,
 * ltkv_append_decode_attention and the per-query pass of planned attention)
 * on this cache. LTKV_ENGINE_AUTO (the default) takes the matrix-core kernel
 * for f16 and Q8_0 pools. LTKV_ENGINE_VALU takes, for f16 pools, the
 * vector-ALU kernels (wave-wide dot products and shuffle reductions, no
 * MFMA: the bandwidth-bound design) that f32 pools always use; the fused
 * append then runs as ltkv_write followed by attention, and group partials
 * are folded by the merge. Results match the reference within the same
 * tolerance either way, and a query's result stays independent of the rest
 * of the batch. Refused (LTKV_ERR_ARG) on Q8_0 pools. No reference
 * counterpart: it keeps the two kernel designs measurable against each
 * other on one build. */
LTKV_API int ltkv_set_attention_engine(ltkv_cache *c, int engine);

/* ---- planned attention (one step descriptor, reused by every layer) ---- */

/* Flags of ltkv_plan_attention. */
#define LTKV_PLAN_SHARED_PREFIX 1u
/* With LTKV_PLAN_SHARED_PREFIX: the grouped (matrix-core) products take Q
 * and the softmax weights rounded to f16, one f16 product each, instead of
 * f16 hi + lo pairs that keep f32 accuracy. Faster grouped attention (half
 * the matrix-core work), at about 3e-4 relative L2 error against the f32
 * computation instead of 1e-7; the per-query pass is unchanged. */
#define LTKV_PLAN_F16_PRODUCTS 2u

/* Plans one batch's attention from the cache's own block tables, the way
 * NativeBackend::decode hands a batch to Model::forward
 * (native/src/lib.rs:163-182, model.rs:431-475): query i reads positions
 * [0, lens[i]) of sequence seqs[i] (lens[i] <= its length; 0 yields zeros).
 * The tables are built on the host and uploaded once, on the cache stream,
 * for every layer's ltkv_planned_attention of the step.
 * With LTKV_PLAN_SHARED_PREFIX, queries whose tables begin with the same
 * blocks (sequences forked by ltkv_share) form groups: the query rows of a
 * group attend to its shared full blocks once, together, on the matrix
 * cores (f16 and q8_0 pools; f32 pools ignore the flag), and each query's own
 * remaining blocks as in ltkv_decode_attention; the two are merged by their
 * softmax statistics. Results agree with ltkv_decode_attention within the
 * attention tolerance (and bit for bit without the flag). A grouped query's
 * summation order depends on its group, so it is not batch-invariant.
 * The plan is invalidated by any later append, truncate, share or
 * init_free_order (ltkv_planned_attention then fails). */
LTKV_API int ltkv_plan_attention(ltkv_cache *c, size_t n, const uint32_t *seqs, const uint32_t *lens,
                        size_t n_heads, size_t head_dim, unsigned flags);

/* Attention of the planned batch on one layer: q [n][n_heads*head_dim] f32
 * (16-byte aligned), out [n][n_heads*head_dim] f32, device pointers. */
LTKV_API int ltkv_planned_attention(ltkv_cache *c, size_t layer, float scale, const float *d_q,
                           float *d_out);

/* Figures of the current plan: out[0] queries, [1] prefix groups, [2]
 * grouped queries, [3] shared blocks (sum over groups), [4] shared-prefix
 * work-groups, [5] table width in blocks. */
LTKV_API int ltkv_plan_stats(const ltkv_cache *c, uint64_t out[6]);

/* ---- resident block tables: the device step descriptor ----------------- */
/* The cache keeps every live sequence's block table in HBM as one row of a
 * [rows][stride] int32 array, plus each row's length in blocks, and uploads
 * only what changed since the last upload: the entries that append (a new
 * block, a copy-on-write replacement), truncate and share touched (the
 * engine's BatchToken / kv_remove / kv_copy traffic, native/src/lib.rs:163-198,
 * scheduler.rs:356-413). No reference counterpart exists: the reference
 * reads its tables in host memory (kv.rs:133-150); here they replace the
 * per-step upload of every query's full table. */

/* Row of each sequence in the resident tables, or -1 for a sequence holding
 * no blocks. A row is assigned when a sequence gets its first block and is
 * reused after the sequence is removed (truncate to 0). Host only; valid for
 * the device after the next upload (which the device ops below enqueue
 * themselves). */
LTKV_API int ltkv_seq_rows(const ltkv_cache *c, size_t n, const uint32_t *seqs, int32_t *rows_out);

/* Enqueues the upload of the table changes made since the last upload, on
 * the cache stream (one small copy of (row, column, block) triples and one
 * kernel). Growing the tables reallocates them and uploads every live row
 * once (the stream is synchronised first). */
LTKV_API int ltkv_sync_tables(ltkv_cache *c);

/* Uploads pending changes, then returns the resident tables: d_tables
 * [n_rows][stride] block ids and d_lengths [n_rows] table lengths in
 * blocks (0 for a free row). Valid until a later call grows them. */
LTKV_API int ltkv_resident_tables(ltkv_cache *c, const int32_t **d_tables, const int32_t **d_lengths,
                                  size_t *stride, size_t *n_rows);

/* Slot mapping of n tokens from the resident tables, on the device: token i
 * at position d_pos[i] of the sequence in row d_rows[i] gets cell
 * block * 16 + pos % 16 (block = its table entry pos / 16, as append
 * returned it, kv.rs:95-121), or -1 when the row is not a live sequence or
 * pos / 16 is past its table. Claim the cells first (ltkv_append_batch);
 * the result feeds ltkv_write / ltkv_write_rope. */
LTKV_API int ltkv_slot_mapping(ltkv_cache *c, size_t n, const int32_t *d_rows, const int64_t *d_pos,
                               int32_t *d_slot_mapping);

/* ltkv_decode_attention over the resident tables: query i reads positions
 * [0, d_lens[i]) of the sequence in row d_rows[i] (device arrays). A row of
 * -1 must come with length 0 (zeros). Same results, bit for bit, as
 * ltkv_decode_attention with that sequence's table. */
LTKV_API int ltkv_decode_attention_rows(ltkv_cache *c, size_t layer, size_t n, size_t n_heads,
                                        size_t head_dim, float scale, const float *d_q,
                                        const int32_t *d_rows, const int32_t *d_lens, float *d_out);

/* Table entries uploaded so far (each (row, column, block) or length update
 * counts one). */
LTKV_API int ltkv_table_uploads(const ltkv_cache *c, uint64_t *entries);

/* ---- host conveniences (synchronous on the stream) --------------------- */

/* Copy the resident tables ([rows][stride] and [rows], the sizes
 * ltkv_resident_tables reports) to host, after pending uploads. */
LTKV_API int ltkv_read_resident_tables(ltkv_cache *c, int32_t *h_tables, int32_t *h_lengths);

/* Copy one layer's K and V pools ([n_blocks][16][kv_dim]) to host: f16 bits,
 * f32, or Q8_0 int8 quants (stored on the device offset by 128, one byte
 * q + 128 each; this copy gives back q). */
LTKV_API int ltkv_read_pool(ltkv_cache *c, size_t layer, void *h_k, void *h_v);

/* Copy one layer's K and V scale pools ([n_blocks][kv_dim/32][16] f16 bits)
 * of a Q8_0 cache to host. */
LTKV_API int ltkv_read_scales(ltkv_cache *c, size_t layer, uint16_t *h_k, uint16_t *h_v);

/* KvCache::rows(layer, seq, n) collected to host [n][kv_dim] buffers. */
LTKV_API int ltkv_rows(ltkv_cache *c, size_t layer, uint32_t seq, size_t n, void *h_k, void *h_v);

/* KvCache::write(layer, block, slot, k, v) (kv.rs:123-131) from host rows. */
LTKV_API int ltkv_write_row(ltkv_cache *c, size_t layer, uint32_t block, uint32_t slot, const float *h_k,
                   const float *h_v);

/* Wait for all work enqueued on the cache's stream, then report (and clear)
 * the faults the device ops met since the last call, which they cannot return
 * themselves (they are asynchronous). Where the reference panics — an index
 * past a sequence's blocks in rows() (kv.rs:147) — a device op instead
 * continues safely and this call returns:
 *   LTKV_ERR_RANGE  a block-table entry outside the pool was read by attention
 *                   (which used block 0 in its place) or by gather (which copied
 *                   nothing for it), or a resident-table row outside the tables
 *                   came with a nonzero length;
 *   LTKV_ERR_ARG    a fused append + attention cell (ltkv_append_decode_attention)
 *                   was not position lens[i] - 1 of query i's table.
 * ltkv_last_error() names the query (or gathered sequence). */
LTKV_API int ltkv_synchronize(ltkv_cache *c);

#ifdef __cplusplus
}
#endif

#endif /* LTKV_H */
