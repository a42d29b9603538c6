// gfx950 (MI355X, CDNA4) kernels of the paged KV-cache path.
//
//   write_kernel / write_q8_kernel      slot-mapped K/V append (kv.rs:123-131 write,
//                                       per model.rs:414-429; q8_0 per quant.rs:785-791)
//   write_rope_kernel / write_rope_q8_kernel  RoPE of K and Q (model.rs:291-308) fused
//                                       into the append
//   copy_blocks_kernel                  copy-on-write block copy (kv.rs:99-110)
//   gather_kernel                       block-table gather (kv.rs:133-150 rows, collected)
//   attn_mfma_kernel                    GQA paged decode attention on the matrix cores
//                                       (f16 and q8_0 pools), split over context partitions
//   attn16_kernel / attn_kernel         the same on the vector ALU (f32 pools)
//   attn_merge_kernel                   log-sum-exp merge of the partitions (model.rs:431-475)
//   mq_attn_kernel                      query rows that share K/V rows (prefix groups,
//                                       prefill chunks) on the matrix cores
//   table_update_kernel / slot_mapping_kernel  resident block tables and the slot
//                                       mapping derived from them
//
// The data-movement kernels are HBM-bandwidth bound and move each byte once
// with 16-byte accesses. Decode attention does ~4-7 flop per KV byte, but
// its per-element work (a G-way dot product per K element, a G-way FMA per
// V element) would keep the vector ALU busy for most of the time the bytes
// take, so it runs its products on MFMA. Wavefronts are 64 lanes;
// reductions use DPP row permutations within a wave.

#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>
#include <type_traits>

#include "ltkv_kernels.h"

// Scratch of the allocation-free decode attention (ltkv_decode_attention_noalloc):
// the partition partials live in this static device array instead of a
// workspace allocated on demand. Each device holds its own copy, at its own
// address, until the process ends. In host code `scratch` names a host-side
// stand-in, not device memory: host code uses only the address that
// hipGetSymbolAddress returns on each device (scratch_address below).
static __device__ __align__(256) uint8_t scratch[ltkv::kScratchBytes];

// Profiling build only (compiled with -DLTKV_TIMELINE into
// libltkv_timeline.so; the product library has none of it): each wave of the
// matrix-core decode kernel records s_memrealtime stamps (100 MHz) of its
// phases in g_timeline[wave of the grid][8], read and cleared by
// ltkv_timeline_read: 0 entry, 1 item found, 2 first tiles' loads issued,
// 3 first tile computed, 4 tile loop done, 5 result written, 6 tiles of the
// item, 7 query << 16 | partition << 8 | first kv head.
#ifdef LTKV_TIMELINE
constexpr int kTimelineWaves = 65536;
static __device__ unsigned long long g_timeline[kTimelineWaves * 8];
#define LTKV_STAMP(i) (tl_[i] = __builtin_amdgcn_s_memrealtime())
#define LTKV_STAMP_ONCE(i) (tl_[i] = tl_[i] ? tl_[i] : __builtin_amdgcn_s_memrealtime())
#else
#define LTKV_STAMP(i) ((void)0)
#define LTKV_STAMP_ONCE(i) ((void)0)
#endif

namespace ltkv {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef __fp16 hf4 __attribute__((__vector_size__(4 * sizeof(__fp16))));
typedef __attribute__((address_space(3))) hf4 lds_hf4;
typedef __attribute__((address_space(3))) char lds_char;

// Fault bits of a cache's status word (reported by ltkv_synchronize).
constexpr int kFaultTable = 1;      // a block-table entry outside the pool
constexpr int kFaultFusedCell = 2;  // a fused append's cell is not position len - 1 of its table

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element
// i % 4 of the 8 bytes addressed by lane 4 j + i / 4 as its element j.
__device__ __forceinline__ hf4 lds_read_tr(const char *p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4f16((lds_hf4 *)(lds_char *)p);
}

// ----------------------------------------------------------------------------
// f32 -> f16, IEEE round-to-nearest-even (the conversion of f16::from_f32).
// v_cvt_f16_f32 rounds to nearest even in the default mode; NaN is rewritten
// explicitly so the result is sign | 0x7e00 | top payload bits on every part.
// ----------------------------------------------------------------------------
__device__ __forceinline__ uint32_t f16_bits(float x) {
  const _Float16 h = (_Float16)x;
  uint32_t b = (uint32_t)__builtin_bit_cast(uint16_t, h);
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  if ((u & 0x7fffffffu) > 0x7f800000u) b = ((u >> 16) & 0x8000u) | 0x7e00u | ((u >> 13) & 0x3ffu);
  return b;
}

__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  return f16_bits(a) | (f16_bits(b) << 16);
}

// ----------------------------------------------------------------------------
// Kernel 1: slot-mapped append. One thread moves 8 consecutive elements of
// ROWS token rows of K and of V: all f32 reads (16 bytes each) are issued
// before the conversions, then one 16-byte f16 write per row and tensor (or
// two 16-byte f32 writes).
//  * sources that fit the caches (the projection that produced K and V just
//    wrote them): one row a thread, plain loads;
//  * STREAM, sources larger than the 256 MB last-level cache: two rows a
//    thread, non-temporal loads (1-2% faster at 64k-262k tokens of kv_dim
//    1024; the same form on a 4216-token step whose sources sat in the
//    caches was 37% slower, the loads missing them).
// ----------------------------------------------------------------------------
// With `order` (ltkv_write_ordered), launch row i is source row order[i] (rows
// outside [0, n_rows) are skipped): a batch's rows taken in ascending cell
// order store into the pool in ascending address order.
// PARTS: 3 writes K and V; 1 only K, 2 only V (the streaming form runs as a
// K launch then a V launch: one read and one write stream per wave instead
// of two each, 1-3% more bandwidth on bulk appends, the same bits).
template <int ELEM, bool STREAM, int PARTS = 3>
__global__ void __launch_bounds__(256)
write_kernel(uint8_t *__restrict__ kpool, uint8_t *__restrict__ vpool,
             const int32_t *__restrict__ slots, const float *__restrict__ k,
             const float *__restrict__ v, int64_t n, int64_t src_stride, int kv_dim,
             int64_t n_slots, const int32_t *__restrict__ order, int64_t n_rows) {
  constexpr int kWriteRows = STREAM ? 2 : 1;
  const int chunks = kv_dim >> 3;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t pair = gid / chunks;
  const int64_t row0 = pair * kWriteRows;
  if (row0 >= n) return;
  const int c = (int)(gid - pair * chunks);
  const int col = c << 3;
  f32x4 a[kWriteRows][4];
  int32_t s[kWriteRows];
#pragma unroll
  for (int j = 0; j < kWriteRows; ++j) {
    int64_t row = row0 + j < n ? row0 + j : row0;  // a missing second row reloads the first
    bool live = row0 + j < n;
    if (order) {
      row = order[row];
      live = live && row >= 0 && row < n_rows;
      row = live ? row : 0;
    }
    s[j] = live ? slots[row] : -1;
    const f32x4 *ks = reinterpret_cast<const f32x4 *>(k + row * src_stride + col);
    const f32x4 *vs = reinterpret_cast<const f32x4 *>(v + row * src_stride + col);
    a[j][0] = a[j][1] = a[j][2] = a[j][3] = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (STREAM) {
      if constexpr ((PARTS & 1) != 0) {
        a[j][0] = __builtin_nontemporal_load(ks);
        a[j][1] = __builtin_nontemporal_load(ks + 1);
      }
      if constexpr ((PARTS & 2) != 0) {
        a[j][2] = __builtin_nontemporal_load(vs);
        a[j][3] = __builtin_nontemporal_load(vs + 1);
      }
    } else {
      if constexpr ((PARTS & 1) != 0) {
        a[j][0] = ks[0];
        a[j][1] = ks[1];
      }
      if constexpr ((PARTS & 2) != 0) {
        a[j][2] = vs[0];
        a[j][3] = vs[1];
      }
    }
  }
#pragma unroll
  for (int j = 0; j < kWriteRows; ++j) {
    if (s[j] < 0 || (int64_t)s[j] >= n_slots) continue;  // skipped cell
    const int64_t dst = (int64_t)s[j] * kv_dim + col;  // cell block*16+slot, token-major row
    if constexpr (ELEM == 2) {
      u32x4 ko, vo;
      ko.x = pack_f16x2(a[j][0].x, a[j][0].y);
      ko.y = pack_f16x2(a[j][0].z, a[j][0].w);
      ko.z = pack_f16x2(a[j][1].x, a[j][1].y);
      ko.w = pack_f16x2(a[j][1].z, a[j][1].w);
      vo.x = pack_f16x2(a[j][2].x, a[j][2].y);
      vo.y = pack_f16x2(a[j][2].z, a[j][2].w);
      vo.z = pack_f16x2(a[j][3].x, a[j][3].y);
      vo.w = pack_f16x2(a[j][3].z, a[j][3].w);
      // non-temporal: the cells are not read again before they leave the
      // caches, and the attention after the append keeps its cache lines
      // (continuous-batching step of 4216 tokens: append 4%, attention 2%
      // faster; bulk appends unchanged)
      if constexpr ((PARTS & 1) != 0) __builtin_nontemporal_store(ko, reinterpret_cast<u32x4 *>(kpool + dst * 2));
      if constexpr ((PARTS & 2) != 0) __builtin_nontemporal_store(vo, reinterpret_cast<u32x4 *>(vpool + dst * 2));
    } else {
      f32x4 *kd = reinterpret_cast<f32x4 *>(kpool + dst * 4);
      f32x4 *vd = reinterpret_cast<f32x4 *>(vpool + dst * 4);
      if constexpr ((PARTS & 1) != 0) {
        kd[0] = a[j][0];
        kd[1] = a[j][1];
      }
      if constexpr ((PARTS & 2) != 0) {
        vd[0] = a[j][2];
        vd[1] = a[j][3];
      }
    }
  }
}

// ----------------------------------------------------------------------------
// Kernel 1 for q8_0 cells: each 32-element group of a K or V row becomes 32
// int8 quants in the cell and its scale d, rounded to f16, in the scale pool
// (the Q8_0 block of quant.rs:188-193: f16 d + 32 int8).
// ----------------------------------------------------------------------------
// DPP move of x (row_mask and bank_mask all set).
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xf, 0xf, false));
}

// quant.rs:785-791 on one 32-element group spread over 4 aligned lanes of
// a wave, 8 elements each (lane j of the group holds elements 8j .. 8j+7):
// amax folded with fmaxf from 0 (a NaN element is skipped, as f32::max; an
// all-NaN group gives 0 as the sequential fold does), then across the 4
// lanes with quad_perm DPP (max is order-free); d = amax / 127, id = 1/d (0
// when d is 0), q = roundf(x * id) (half away from zero) saturated to int8
// with NaN -> 0 (Rust's `as i8`); every lane stores its 8 quants, lane 0 d
// as f16. Quants are stored offset by 128 (byte q + 128, so int8 -128..127
// is 0..255): the readers turn a byte into an f16 without a sign fix-up.
__device__ __forceinline__ void quantize_store4(const float (&x)[8], int j, int8_t *__restrict__ dq,
                                                uint16_t *__restrict__ ds) {
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = __builtin_fmaxf(amax, __builtin_fabsf(x[i]));
  amax = __builtin_fmaxf(amax, dpp<0xB1>(amax));  // quad_perm [1,0,3,2]: lane ^ 1
  amax = __builtin_fmaxf(amax, dpp<0x4E>(amax));  // quad_perm [2,3,0,1]: lane ^ 2
  const float d = amax / 127.f;
  const float id = d > 0.f ? 1.f / d : 0.f;
  uint32_t w[2] = {0, 0};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float r = __builtin_roundf(x[i] * id);  // half away from zero
    int qv = 0;
    if (r == r) qv = r > 127.f ? 127 : (r < -128.f ? -128 : (int)r);
    w[i >> 2] |= (uint32_t)((qv + 128) & 0xff) << (8 * (i & 3));
  }
  *reinterpret_cast<u32x2 *>(dq + 8 * j) = u32x2{w[0], w[1]};
  if (j == 0) *ds = (uint16_t)f16_bits(d);
}

// Scale entry of (cell s, group g): layout [block][kv_dim / 32][16 slots],
// so the scales of one kv head of a block are one contiguous run.
__device__ __forceinline__ int64_t scale_index(int32_t s, int g, int kg) {
  return (((int64_t)(s >> 4) * kg + g) << 4) + (s & 15);
}

// Kernel 1 for q8_0 cells: 4 lanes per 32-element group of K or V, two
// 16-byte loads and one 8-byte store per lane.
__global__ void __launch_bounds__(256)
write_q8_kernel(int8_t *__restrict__ kpool, int8_t *__restrict__ vpool, uint16_t *__restrict__ kscale,
                uint16_t *__restrict__ vscale, const int32_t *__restrict__ slots,
                const float *__restrict__ k, const float *__restrict__ v, int64_t n, int64_t src_stride,
                int kv_dim, int64_t n_slots, const int32_t *__restrict__ order, int64_t n_rows) {
  const int e8 = kv_dim >> 3;  // 8-element eighths of a K (or V) row
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t i = gid / (2 * e8);
  if (i >= n) return;  // whole 4-lane groups leave together (2 e8 is a multiple of 4)
  const int u = (int)(gid - i * 2 * e8);
  const int64_t row = order ? order[i] : i;  // write_kernel's order
  if (order && (row < 0 || row >= n_rows)) return;
  const int32_t s = slots[row];
  if (s < 0 || (int64_t)s >= n_slots) return;
  const bool is_v = u >= e8;
  const int e = (is_v ? u - e8 : u) << 3;  // element offset in the row
  const f32x4 *src = reinterpret_cast<const f32x4 *>((is_v ? v : k) + row * src_stride + e);
  const f32x4 t0 = src[0], t1 = src[1];
  const float x[8] = {t0.x, t0.y, t0.z, t0.w, t1.x, t1.y, t1.z, t1.w};
  quantize_store4(x, (e >> 3) & 3, (is_v ? vpool : kpool) + (int64_t)s * kv_dim + (e & ~31),
                  (is_v ? vscale : kscale) + scale_index(s, e >> 5, kv_dim >> 5));
}

// ----------------------------------------------------------------------------
// Kernel 1 fused with RoPE (model.rs:291-308 then kv.rs:123-131): one launch
// rotates Q in place and K on its way into the pool, and appends V. A thread
// owns one unit of a head: 4 rotation pairs (8 elements: (2i, 2i+1) pairs
// adjacent, or NeoX pairs (i, i + rope_dim/2) as 4 + 4) or 8 unrotated
// elements past rope_dim. cos/sin come from the host-built table (the same
// libm the reference calls), and the products are not contracted into FMAs
// (rustc does not contract), so the results are bit-identical.
// ----------------------------------------------------------------------------
__device__ __forceinline__ void rope_pairs(const float *__restrict__ cs, float (&x0)[4], float (&x1)[4]) {
#pragma clang fp contract(off)
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const float c = cs[2 * p], sn = cs[2 * p + 1];
    const float a = x0[p], b = x1[p];
    x0[p] = a * c - b * sn;
    x1[p] = a * sn + b * c;
  }
}

// One unit of a head row (4 rotation pairs, or 8 unrotated elements past
// rope_dim): its element offsets e0 .. e0+3 and e1 .. e1+3 within the head
// and the rotated values in o.
__device__ __forceinline__ void rope_unit(const float *__restrict__ head, int w, int pos,
                                          const float *__restrict__ table, int rope_dim, int neox,
                                          int &e0, int &e1, float (&o)[8]) {
  const int upr = rope_dim >> 3;
  if (w >= upr) {  // past rope_dim: unrotated
    e0 = (upr << 3) + ((w - upr) << 3);
    e1 = e0 + 4;
  } else if (neox) {
    e0 = w << 2;
    e1 = e0 + (rope_dim >> 1);
  } else {
    e0 = w << 3;
    e1 = e0 + 4;
  }
  const f32x4 a = *reinterpret_cast<const f32x4 *>(head + e0);
  const f32x4 b = *reinterpret_cast<const f32x4 *>(head + e1);
  o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
  o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  if (w < upr) {
    const float *cs = table + ((int64_t)pos * (rope_dim >> 1)) * 2;
    if (neox) {  // pairs (e0 + p, e1 + p), pair index e0 + p
      float x0[4] = {o[0], o[1], o[2], o[3]}, x1[4] = {o[4], o[5], o[6], o[7]};
      rope_pairs(cs + 2 * e0, x0, x1);
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        o[p] = x0[p];
        o[4 + p] = x1[p];
      }
    } else {  // pairs (e0 + 2p, e0 + 2p + 1), pair index e0 / 2 + p
      float x0[4] = {o[0], o[2], o[4], o[6]}, x1[4] = {o[1], o[3], o[5], o[7]};
      rope_pairs(cs + e0, x0, x1);
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        o[2 * p] = x0[p];
        o[2 * p + 1] = x1[p];
      }
    }
  }
}

template <int ELEM>
__global__ void __launch_bounds__(256)
write_rope_kernel(uint8_t *__restrict__ kpool, uint8_t *__restrict__ vpool,
                  const int32_t *__restrict__ slots, const int32_t *__restrict__ positions,
                  const float *__restrict__ k, const float *__restrict__ v, float *__restrict__ q,
                  int64_t n, int64_t src_stride, int64_t q_stride, int kv_dim, int n_kv_heads,
                  int n_heads, int64_t n_slots, const float *__restrict__ table, int max_pos,
                  int rope_dim, int head_dim, int neox) {
  const int uph = head_dim >> 3;          // units per head
  const int ku = n_kv_heads * uph;        // K units per token
  const int vu = kv_dim >> 3;             // V units per token
  const int qu = q ? n_heads * uph : 0;   // Q units per token
  const int per = ku + vu + qu;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = gid / per;
  if (row >= n) return;
  int u = (int)(gid - row * per);
  const int32_t pos = positions[row];
  if (pos < 0 || pos >= max_pos) return;
  const int32_t s = slots[row];
  const bool cell = s >= 0 && (int64_t)s < n_slots;
  if (u >= ku && u < ku + vu) {  // V: plain append of 8 elements
    if (!cell) return;
    const int col = (u - ku) << 3;
    const f32x4 *vs = reinterpret_cast<const f32x4 *>(v + row * src_stride + col);
    const f32x4 v0 = vs[0], v1 = vs[1];
    const int64_t dst = (int64_t)s * kv_dim + col;
    if constexpr (ELEM == 2) {
      u32x4 vo;
      vo.x = pack_f16x2(v0.x, v0.y);
      vo.y = pack_f16x2(v0.z, v0.w);
      vo.z = pack_f16x2(v1.x, v1.y);
      vo.w = pack_f16x2(v1.z, v1.w);
      *reinterpret_cast<u32x4 *>(vpool + dst * 2) = vo;
    } else {
      f32x4 *vd = reinterpret_cast<f32x4 *>(vpool + dst * 4);
      vd[0] = v0;
      vd[1] = v1;
    }
    return;
  }
  const bool is_q = u >= ku + vu;
  if (!is_q && !cell) return;
  if (is_q) u -= ku + vu;
  const int h = u / uph, w = u - h * uph;
  const float *src = is_q ? q + row * q_stride : k + row * src_stride;
  const int hb = h * head_dim;
  int e0, e1;
  float o[8];
  rope_unit(src + hb, w, pos, table, rope_dim, neox, e0, e1, o);
  if (is_q) {
    float *qd = q + row * q_stride + hb;
    *reinterpret_cast<f32x4 *>(qd + e0) = f32x4{o[0], o[1], o[2], o[3]};
    *reinterpret_cast<f32x4 *>(qd + e1) = f32x4{o[4], o[5], o[6], o[7]};
    return;
  }
  const int64_t dst = (int64_t)s * kv_dim + hb;
  if constexpr (ELEM == 2) {
    uint16_t *kd = reinterpret_cast<uint16_t *>(kpool) + dst;
    *reinterpret_cast<u32x2 *>(kd + e0) = u32x2{pack_f16x2(o[0], o[1]), pack_f16x2(o[2], o[3])};
    *reinterpret_cast<u32x2 *>(kd + e1) = u32x2{pack_f16x2(o[4], o[5]), pack_f16x2(o[6], o[7])};
  } else {
    float *kd = reinterpret_cast<float *>(kpool) + dst;
    *reinterpret_cast<f32x4 *>(kd + e0) = f32x4{o[0], o[1], o[2], o[3]};
    *reinterpret_cast<f32x4 *>(kd + e1) = f32x4{o[4], o[5], o[6], o[7]};
  }
}

// ----------------------------------------------------------------------------
// Kernel 1 with RoPE for q8_0 cells: 4 lanes per 32-element group of K
// (rotated, then quantised as write_q8_kernel) or of V (quantised), 8
// elements a lane; and a thread per 8-element unit of Q (rotated in place,
// as write_rope_kernel). A lane's K elements rotate with the products of
// rope_pairs, 4 at a time: (2i, 2i+1) partners lie in the lane, NeoX
// partners (i, i + rope_dim/2) are the 4 elements rope_dim/2 away (rope_dim
// is a multiple of 8, so each 4 lie on one side).
// ----------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
write_rope_q8_kernel(int8_t *__restrict__ kpool, int8_t *__restrict__ vpool, uint16_t *__restrict__ kscale,
                     uint16_t *__restrict__ vscale, const int32_t *__restrict__ slots,
                     const int32_t *__restrict__ positions, const float *__restrict__ k,
                     const float *__restrict__ v, float *__restrict__ q, int64_t n, int64_t src_stride,
                     int64_t q_stride, int kv_dim, int n_heads, int64_t n_slots,
                     const float *__restrict__ table, int max_pos, int rope_dim, int head_dim, int neox) {
#pragma clang fp contract(off)
  const int e8 = kv_dim >> 3;             // 8-element eighths of a K (or V) row
  const int uph = head_dim >> 3;          // Q units per head
  const int qu = q ? n_heads * uph : 0;   // Q units per token
  // Threads [0, n * 2 e8) take the K/V eighths, the rest the Q units, so a
  // wave runs one of the two paths.
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t n_kv = n * 2 * e8;
  const bool q_unit = gid >= n_kv;
  const int64_t row = q_unit ? (gid - n_kv) / (qu > 0 ? qu : 1) : gid / (2 * e8);
  if (row >= n || (q_unit && qu == 0)) return;
  const int u = (int)(q_unit ? gid - n_kv - row * qu : gid - row * 2 * e8);
  const int32_t pos = positions[row];
  if (pos < 0 || pos >= max_pos) return;  // uniform over a token's 4-lane groups
  if (q_unit) {  // Q unit: rotated in place
    const int h = u / uph, w = u - h * uph;
    float *qh = q + row * q_stride + (int64_t)h * head_dim;
    int e0, e1;
    float o[8];
    rope_unit(qh, w, pos, table, rope_dim, neox, e0, e1, o);
    *reinterpret_cast<f32x4 *>(qh + e0) = f32x4{o[0], o[1], o[2], o[3]};
    *reinterpret_cast<f32x4 *>(qh + e1) = f32x4{o[4], o[5], o[6], o[7]};
    return;
  }
  const int32_t s = slots[row];
  if (s < 0 || (int64_t)s >= n_slots) return;
  const bool is_v = u >= e8;
  const int e = (is_v ? u - e8 : u) << 3;  // element offset in the row
  const float *src = (is_v ? v : k) + row * src_stride;
  const f32x4 t0 = *reinterpret_cast<const f32x4 *>(src + e), t1 = *reinterpret_cast<const f32x4 *>(src + e + 4);
  float x[8] = {t0.x, t0.y, t0.z, t0.w, t1.x, t1.y, t1.z, t1.w};
  if (!is_v) {
    const int h = e / head_dim, eh0 = e - h * head_dim;  // head and offset in it
    if (eh0 < rope_dim) {  // rope_dim is a multiple of 8: all 8 elements rotate
      const float *cs = table + ((int64_t)pos * (rope_dim >> 1)) * 2;
      const int half = rope_dim >> 1;
#pragma unroll
      for (int qd = 0; qd < 2; ++qd) {  // the lane's two quads of 4 elements
        const int eh = eh0 + 4 * qd;
        if (neox) {
          const bool lo = eh < half;  // first (lo) or second member of its pairs
          const f32x4 pt = *reinterpret_cast<const f32x4 *>(src + e + 4 * qd + (lo ? half : -half));
          const float pr[4] = {pt.x, pt.y, pt.z, pt.w};
          const int i0 = lo ? eh : eh - half;  // pair index of the quad's element 0
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float c = cs[2 * (i0 + i)], sn = cs[2 * (i0 + i) + 1];
            x[4 * qd + i] = lo ? x[4 * qd + i] * c - pr[i] * sn : pr[i] * sn + x[4 * qd + i] * c;
          }
        } else {
#pragma unroll
          for (int i = 0; i < 4; i += 2) {  // pair (eh + i, eh + i + 1), index (eh + i) / 2
            const float c = cs[eh + i], sn = cs[eh + i + 1];
            const float a = x[4 * qd + i], b = x[4 * qd + i + 1];
            x[4 * qd + i] = a * c - b * sn;
            x[4 * qd + i + 1] = a * sn + b * c;
          }
        }
      }
    }
  }
  quantize_store4(x, (e >> 3) & 3, (is_v ? vpool : kpool) + (int64_t)s * kv_dim + (e & ~31),
                  (is_v ? vscale : kscale) + scale_index(s, e >> 5, kv_dim >> 5));
}
// ----------------------------------------------------------------------------
// Kernel 2: block copy. Work item = one chunk of THREADS x VEC 16-byte
// vectors of one (pair, layer, tensor); every thread issues its VEC
// non-temporal loads before its stores. Two forms:
//  * claim batches (copy-on-write, typically up to a few hundred pairs):
//    256 threads x 2 vectors (8 KiB chunks), the layers of a pair adjacent,
//    plain stores.
//    At the 255-copy step of 256 forks (one shared source block) 8 KiB
//    chunks ran 5.2-5.4 us against 5.6-5.8 us for 16 KiB, 6.4-6.5 for 4 KiB
//    and 7.2-7.3 for 32 KiB; 1024-thread work-groups 20% slower.
//  * bulk batches (4096 pairs and more): 1024 threads x 1 vector (16 KiB
//    chunks), layer the slowest index, so the work-groups in flight copy
//    consecutive pairs of one layer, in the destination order set up by
//    copy_order_* below; non-temporal stores.
// The order in which work-groups write matters on this part: 131 072 copies
// of 32 KiB blocks between random places ran at 64% of 8 TB/s issued in a
// random destination order and at 74% issued in ascending destination order
// (the same with the destinations only bucketed by 64 blocks), so the
// claim's copy-on-write pairs are sorted by destination on the host and bulk
// caller batches are bucketed by destination on the device first.
// ----------------------------------------------------------------------------
constexpr int kCopyBulkThreads = 1024;

template <int THREADS, int VEC, bool LAYER_MAJOR>
__global__ void __launch_bounds__(THREADS)
copy_blocks_kernel(uint8_t *__restrict__ kpool, uint8_t *__restrict__ vpool,
                   const int32_t *__restrict__ pairs, int64_t n_pairs, int n_layers, int64_t n_blocks,
                   int64_t block_bytes, int64_t layer_bytes, int chunks_per_block) {
  int64_t wg = blockIdx.x;
  const int chunk = (int)(wg % chunks_per_block);
  wg /= chunks_per_block;
  const int tensor = (int)(wg & 1);
  wg >>= 1;
  const int64_t pair = LAYER_MAJOR ? wg % n_pairs : wg / n_layers;
  const int64_t layer = LAYER_MAJOR ? wg / n_pairs : wg % n_layers;
  const int32_t src = pairs[2 * pair], dst = pairs[2 * pair + 1];
  if (src < 0 || dst < 0 || src >= n_blocks || dst >= n_blocks || src == dst) return;
  uint8_t *base = (tensor ? vpool : kpool) + layer * layer_bytes;
  const u32x4 *s = reinterpret_cast<const u32x4 *>(base + (int64_t)src * block_bytes);
  u32x4 *d = reinterpret_cast<u32x4 *>(base + (int64_t)dst * block_bytes);
  const int64_t n16 = block_bytes >> 4;
  const int64_t i0 = (int64_t)chunk * THREADS * VEC + threadIdx.x;
  u32x4 r[VEC];
#pragma unroll
  for (int u = 0; u < VEC; ++u) {
    const int64_t i = i0 + u * THREADS;
    if (i < n16) r[u] = __builtin_nontemporal_load(s + i);
  }
#pragma unroll
  for (int u = 0; u < VEC; ++u) {
    const int64_t i = i0 + u * THREADS;
    if (i >= n16) continue;
    if constexpr (LAYER_MAJOR) __builtin_nontemporal_store(r[u], d + i);
    else d[i] = r[u];
  }
}

// Destination buckets of 2^kCopyOrderShift blocks: a counting sort of the
// pairs by bucket (count, exclusive scan, scatter). The order within a
// bucket is whatever the atomics give; it changes no result, since every
// destination of a batch is written by one pair only. `counts` is all zero
// on entry and is left all zero by copy_order_scan.
constexpr int kCopyOrderShift = 6;

__device__ __forceinline__ int32_t copy_bucket(int32_t dst, int64_t n_blocks) {
  return (dst < 0 || dst >= n_blocks) ? 0 : (dst >> kCopyOrderShift);
}

__global__ void __launch_bounds__(256)
copy_order_count(const int32_t *__restrict__ pairs, int64_t n, int64_t n_blocks,
                 int32_t *__restrict__ counts) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  atomicAdd(counts + copy_bucket(pairs[2 * i + 1], n_blocks), 1);
}

// One work-group: cursors = exclusive prefix sums of counts; counts cleared.
__global__ void __launch_bounds__(1024)
copy_order_scan(int32_t *__restrict__ counts, int32_t *__restrict__ cursors, int n_buckets) {
  __shared__ int32_t sh[1024];
  int32_t carry = 0;
  for (int base = 0; base < n_buckets; base += 1024) {
    const int i = base + (int)threadIdx.x;
    const int32_t c = i < n_buckets ? counts[i] : 0;
    sh[threadIdx.x] = c;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {  // inclusive Hillis-Steele scan
      const int32_t t = threadIdx.x >= (unsigned)off ? sh[threadIdx.x - off] : 0;
      __syncthreads();
      sh[threadIdx.x] += t;
      __syncthreads();
    }
    if (i < n_buckets) {
      cursors[i] = carry + sh[threadIdx.x] - c;
      counts[i] = 0;
    }
    carry += sh[1023];
    __syncthreads();
  }
}

__global__ void __launch_bounds__(256)
copy_order_scatter(const int32_t *__restrict__ pairs, int64_t n, int64_t n_blocks,
                   int32_t *__restrict__ cursors, int32_t *__restrict__ sorted) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int32_t src = pairs[2 * i], dst = pairs[2 * i + 1];
  const int32_t pos = atomicAdd(cursors + copy_bucket(dst, n_blocks), 1);
  if (pos < 0 || pos >= n) return;  // only if counts were not zero on entry
  sorted[2 * (int64_t)pos] = src;
  sorted[2 * (int64_t)pos + 1] = dst;
}

// ----------------------------------------------------------------------------
// Kernel 3: gather. Work-group = (sequence, table entry, K or V, 16 KiB chunk
// of the block): the valid rows of one block are one contiguous run in the
// token-major layout, in source and destination, so each thread moves one
// 16-byte vector. Small work-groups with one load per thread keep the most
// loads in flight across the chip (measured faster than fewer, longer
// work-groups on this scatter pattern).
// ----------------------------------------------------------------------------
constexpr int kGatherThreads = 1024;
constexpr int64_t kGatherChunk = kGatherThreads;  // 16-byte vectors per work-group

__global__ void __launch_bounds__(kGatherThreads)
gather_kernel(const uint8_t *__restrict__ kpool, const uint8_t *__restrict__ vpool,
              const int32_t *__restrict__ tables, int64_t table_stride,
              const int32_t *__restrict__ lens, const int64_t *__restrict__ out_offsets,
              uint8_t *__restrict__ kout, uint8_t *__restrict__ vout, int64_t n_blocks,
              int64_t row_bytes, int chunks, int32_t *__restrict__ status) {
  const int64_t per_entry = 2 * (int64_t)chunks;
  const int64_t entry = blockIdx.x / per_entry;
  const int part = (int)(blockIdx.x - entry * per_entry);
  const int is_v = part >= chunks;
  const int chunk = part - is_v * chunks;
  const int64_t seq = entry / table_stride;
  const int64_t j = entry - seq * table_stride;
  int64_t len = lens[seq];
  if (len > table_stride * 16) len = table_stride * 16;
  const int64_t start = j * 16;
  if (start >= len) return;
  const int64_t rows = len - start < 16 ? len - start : 16;
  const int32_t blk = tables[seq * table_stride + j];
  if (blk < 0 || blk >= n_blocks) {  // kv.rs:147 panics here; nothing is copied
    if (threadIdx.x == 0 && status) {
      __hip_atomic_fetch_or(status, kFaultTable, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      status[1] = (int32_t)seq;
    }
    return;
  }
  const int64_t i = (int64_t)chunk * kGatherChunk + threadIdx.x;
  if (i >= (rows * row_bytes) >> 4) return;
  const u32x4 *src = reinterpret_cast<const u32x4 *>((is_v ? vpool : kpool) +
                                                     (int64_t)blk * 16 * row_bytes);
  u32x4 *dst = reinterpret_cast<u32x4 *>((is_v ? vout : kout) + (out_offsets[seq] + start) * row_bytes);
  __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

// ----------------------------------------------------------------------------
// Kernel 4: GQA paged decode attention, VALU form (f32 pools; f16 and q8_0
// pools take attn_mfma_kernel below).
//
// Work-group = 4 waves on (query, kv head, context partition). The waves take
// the partition's blocks round-robin. For one block a wave reads the head's
// 16 x head_dim K tile and V tile with 16-byte loads: L lanes cover one row,
// so a wave load covers 64/L rows. Each lane keeps the g query heads of its
// column slice in registers (pre-scaled by scale*log2 e) and computes partial
// dots; a DPP butterfly over the L lanes finishes each score. Online softmax
// (exp2 domain) runs per row group, so no cross-row-group traffic happens in
// the block loop; row groups, then waves (through LDS) are merged once at the
// end. With one partition the work-group writes the normalised output, else
// it writes (numerator, max, sum) for attn_merge_kernel.
// ----------------------------------------------------------------------------

// Sum over each aligned group of L lanes (L in 4..32); every lane gets it.
template <int L>
__device__ __forceinline__ float group_sum(float x) {
  x += dpp<0xB1>(x);  // quad_perm [1,0,3,2]
  x += dpp<0x4E>(x);  // quad_perm [2,3,0,1]
  if constexpr (L >= 8) x += dpp<0x141>(x);  // row_half_mirror
  if constexpr (L >= 16) x += dpp<0x140>(x); // row_mirror
  if constexpr (L >= 32) x += __shfl_xor(x, 16);
  return x;
}

// Element tile of the VALU decode kernels (f32 pools): 4 elements per
// 16-byte load.
template <typename T>
struct Tile;

template <>
struct Tile<_Float16> {
  static constexpr int E = 8;  // elements per 16-byte load
  __device__ static __forceinline__ void unpack(const u32x4 &u, float (&f)[8]) {
    const h8 h = __builtin_bit_cast(h8, u);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = (float)h[i];
  }
};

template <>
struct Tile<float> {
  static constexpr int E = 4;
  __device__ static __forceinline__ void unpack(const u32x4 &u, float (&f)[4]) {
    const f32x4 v = __builtin_bit_cast(f32x4, u);
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = v[i];
  }
};

constexpr int kAttnWaves = 4;
constexpr int kBufferWord3 = 0x00020000;  // buffer descriptor word 3 for gfx9-family raw buffers
constexpr int kNt = 2;                    // buffer load cache policy: non-temporal
constexpr float kLog2e = 1.4426950408889634f;

// Block table of query qi: row qi of `tables`, or, with resident tables, row
// rows[qi] (a row outside [0, n_rows) reads row 0: such a query must have
// length 0, and nothing is read then).
__device__ __forceinline__ const int32_t *table_of(const int32_t *tables, int64_t stride,
                                                   const int32_t *rows, int64_t n_rows, int64_t qi) {
  int64_t r = qi;
  if (rows) {
    r = ((const __attribute__((address_space(4))) int32_t *)rows)[qi];  // uniform: the scalar cache
    if (r < 0 || r >= n_rows) r = 0;
  }
  return tables + r * stride;
}

// Faults a device op met, for ltkv_synchronize to report (the reference
// panics at the same places): status[0] ORs the fault bits, status[1] holds
// the query of one of them. The op goes on safely (a bad entry reads block
// 0), so nothing faults on the GPU.
// A wave-uniform read of memory no thread writes during the launch (block
// tables, lengths), through the scalar cache: the constant address space
// tells the compiler so, where stores elsewhere in the kernel would keep it
// from proving it.
__device__ __forceinline__ int32_t scalar_read(const int32_t *p, int64_t i) {
  return ((const __attribute__((address_space(4))) int32_t *)p)[i];
}

// Every calling lane stores the same bits and query: no lane test, so values
// the caller computes around a report stay uniform over the wave.
__device__ __forceinline__ void report_fault(int32_t *status, int code, int64_t qi) {
  if (!status) return;
  __hip_atomic_fetch_or(status, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  status[1] = (int32_t)qi;
}

// Checks the table entries of blocks [b0, b1) (the positions a work-group
// reads: kv.rs:147 indexes the sequence's blocks with them) and the query's
// row in the resident tables; run once before the tile loop, one wave.
__device__ __forceinline__ void check_table(const int32_t *tab, int b0, int b1, int64_t n_blocks,
                                            const int32_t *rows, int64_t n_rows, int64_t qi, int32_t *status) {
  if (!status || b1 <= b0) return;
  bool bad = false;
  if (rows) {
    const int32_t r = rows[qi];
    bad = r < 0 || r >= n_rows;  // such a query must have length 0
  }
  for (int b = b0 + (int)(threadIdx.x & 63); b < b1 && !bad; b += 64) {
    const int32_t blk = tab[b];
    bad = blk < 0 || blk >= n_blocks;
  }
  if (__builtin_amdgcn_ballot_w64(bad)) report_fault(status, kFaultTable, qi);
}

template <typename T, int HD, int G>
__global__ void __launch_bounds__(256)
attn_kernel(const T *__restrict__ kpool, const T *__restrict__ vpool, const float *__restrict__ q,
            const int32_t *__restrict__ tables, int64_t table_stride,
            const int32_t *__restrict__ lens, float *__restrict__ out, float *__restrict__ part_o,
            float *__restrict__ part_ml, int n_kv_heads, int64_t n_blocks, int64_t block_stride,
            int64_t slot_stride, int64_t head_stride, float qscale, int part_tokens,
            int max_parts, const int32_t *__restrict__ pre_parts,
            const int32_t *__restrict__ qmap, const int32_t *__restrict__ rows, int64_t n_rows,
            int64_t max_len, int32_t *__restrict__ status) {
  constexpr int E = Tile<T>::E;
  constexpr int L = HD / E;        // lanes per row
  constexpr int RPL = 64 / L;      // rows per wave load
  constexpr int LOADS = 16 / RPL;  // wave loads per 16-row tile
  static_assert(L >= 4 && L <= 32 && LOADS >= 1, "unsupported head_dim / dtype");

  // 1-D grid, kv head fastest: the work-groups reading the same blocks of a
  // query (one per kv head) are dispatched together.
  const int kvh = (int)(blockIdx.x % n_kv_heads);
  const int part = (int)((blockIdx.x / n_kv_heads) % max_parts);
  const int64_t qx = blockIdx.x / ((unsigned)n_kv_heads * max_parts);
  const int64_t qi = qmap ? qmap[qx] : qx;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane % L, rg = lane / L;
  const int n_heads = n_kv_heads * G;

  int64_t len = lens[qi];
  if (len < 0) len = 0;
  if (len > max_len) len = max_len;
  // A query with group partials and nothing else to read (or whose group
  // wrote its output) has no work here.
  if (pre_parts && (pre_parts[qi] < 0 || (pre_parts[qi] > 0 && len == 0))) return;
  const int pt = partition_tokens(len, part_tokens);
  const int np = len > 0 ? (int)((len + pt - 1) / pt) : 1;
  if (part >= np) return;  // uniform over the work-group
  const int64_t tok0 = (int64_t)part * pt;
  const int64_t tok1 = len < tok0 + pt ? len : tok0 + pt;
  const int b0 = (int)(tok0 >> 4), b1 = (int)((tok1 + 15) >> 4);

  float qv[G][E];
  {
    const float *qp = q + qi * (int64_t)n_heads * HD + (int64_t)kvh * G * HD + c * E;
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int e = 0; e < E; e += 4) {
        const f32x4 t = *reinterpret_cast<const f32x4 *>(qp + h * HD + e);
        qv[h][e] = t.x * qscale;
        qv[h][e + 1] = t.y * qscale;
        qv[h][e + 2] = t.z * qscale;
        qv[h][e + 3] = t.w * qscale;
      }
  }

  float m[G], l[G], acc[G][E];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) acc[h][e] = 0.f;
  }

  const int32_t *tab = table_of(tables, table_stride, rows, n_rows, qi);
  check_table(tab, b0, b1, n_blocks, rows, n_rows, qi, status);
  const int64_t lane_off = (int64_t)rg * slot_stride + c * E;
  const int64_t head_off = (int64_t)kvh * head_stride;

  auto load_tile = [&](int b, u32x4 (&kr)[LOADS], u32x4 (&vr)[LOADS]) {
    int32_t blk = tab[b];
    if (blk < 0 || blk >= n_blocks) blk = 0;  // out-of-range entries read block 0 (never faults)
    const int64_t base = (int64_t)blk * block_stride + head_off + lane_off;
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      const int64_t o = base + (int64_t)j * RPL * slot_stride;
      kr[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(kpool + o));
      vr[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(vpool + o));
    }
  };

  auto compute_tile = [&](int b, const u32x4 (&kr)[LOADS], const u32x4 (&vr)[LOADS]) {
    const int valid = (int)(tok1 - (int64_t)b * 16);  // rows of this tile inside the context
    float s[LOADS][G];
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      float kf[E];
      Tile<T>::unpack(kr[j], kf);
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float a = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) a = __builtin_fmaf(qv[h][e], kf[e], a);
        s[j][h] = group_sum<L>(a);
      }
    }
    if (valid < 16) {
#pragma unroll
      for (int j = 0; j < LOADS; ++j)
        if (rg + j * RPL >= valid)
#pragma unroll
          for (int h = 0; h < G; ++h) s[j][h] = -INFINITY;
    }
    float p[LOADS][G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float bm = s[0][h];
#pragma unroll
      for (int j = 1; j < LOADS; ++j) bm = __builtin_fmaxf(bm, s[j][h]);
      const float mn = __builtin_fmaxf(m[h], bm);
      const float mref = mn == -INFINITY ? 0.f : mn;
      const float alpha = __builtin_amdgcn_exp2f(m[h] - mref);
      float ps = 0.f;
#pragma unroll
      for (int j = 0; j < LOADS; ++j) {
        p[j][h] = __builtin_amdgcn_exp2f(s[j][h] - mref);
        ps += p[j][h];
      }
      l[h] = l[h] * alpha + ps;
      m[h] = mn;
#pragma unroll
      for (int e = 0; e < E; ++e) acc[h][e] *= alpha;
    }
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      float vf[E];
      Tile<T>::unpack(vr[j], vf);
      if (valid < 16 && rg + j * RPL >= valid) {
#pragma unroll
        for (int e = 0; e < E; ++e) vf[e] = 0.f;  // stale slots may hold non-finite bits
      }
#pragma unroll
      for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < E; ++e) acc[h][e] = __builtin_fmaf(p[j][h], vf[e], acc[h][e]);
    }
  };

  // Software pipeline: the next tile's loads are in flight while the current
  // one is computed. Past the end the prefetch re-reads the current tile
  // (cache hit) so the wait counts stay static.
  {
    u32x4 ka[LOADS], va[LOADS], kb[LOADS], vb[LOADS];
    int b = b0 + wave;
    if (b < b1) load_tile(b, ka, va);
    while (b < b1) {
      const int bn = b + kAttnWaves < b1 ? b + kAttnWaves : b;
      load_tile(bn, kb, vb);
      compute_tile(b, ka, va);
      b += kAttnWaves;
      if (b >= b1) break;
      const int bn2 = b + kAttnWaves < b1 ? b + kAttnWaves : b;
      load_tile(bn2, ka, va);
      compute_tile(b, kb, vb);
      b += kAttnWaves;
    }
  }

  // Merge the row groups of the wave (lanes L, 2L, .. apart hold the same column).
#pragma unroll
  for (int off = L; off < 64; off <<= 1) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float mo = __shfl_xor(m[h], off);
      const float lo = __shfl_xor(l[h], off);
      const float mn = __builtin_fmaxf(m[h], mo);
      const float mref = mn == -INFINITY ? 0.f : mn;
      const float as = __builtin_amdgcn_exp2f(m[h] - mref);
      const float ao = __builtin_amdgcn_exp2f(mo - mref);
      l[h] = l[h] * as + lo * ao;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float other = __shfl_xor(acc[h][e], off);
        acc[h][e] = acc[h][e] * as + other * ao;
      }
      m[h] = mn;
    }
  }

  // Merge the waves through LDS.
  __shared__ float sm_acc[kAttnWaves][G][HD];
  __shared__ float sm_m[kAttnWaves][G], sm_l[kAttnWaves][G];
  if (rg == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
#pragma unroll
      for (int e = 0; e < E; ++e) sm_acc[wave][h][c * E + e] = acc[h][e];
      if (c == 0) {
        sm_m[wave][h] = m[h];
        sm_l[wave][h] = l[h];
      }
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < G * HD; idx += 256) {
    const int h = idx / HD, d = idx - h * HD;
    float mx = sm_m[0][h];
#pragma unroll
    for (int w = 1; w < kAttnWaves; ++w) mx = __builtin_fmaxf(mx, sm_m[w][h]);
    const float mref = mx == -INFINITY ? 0.f : mx;
    float lsum = 0.f, o = 0.f;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) {
      const float a = __builtin_amdgcn_exp2f(sm_m[w][h] - mref);
      lsum += sm_l[w][h] * a;
      o += sm_acc[w][h][d] * a;
    }
    const int64_t qh = qi * n_heads + (int64_t)kvh * G + h;
    if (np == 1 && !(pre_parts && pre_parts[qi] > 0)) {  // else merged with prefix partials
      out[qh * HD + d] = lsum > 0.f ? o / lsum : 0.f;
    } else {
      const int64_t pi = qh * max_parts + part;
      part_o[pi * HD + d] = o;
      if (d == 0) {
        part_ml[2 * pi] = mx;
        part_ml[2 * pi + 1] = lsum;
      }
    }
  }
}

// Merge of the context partitions of one (query, head): O = sum_p o_p 2^(m_p-M),
// L = sum_p l_p 2^(m_p-M), out = O / L. A (query, head) pair takes HD/4
// threads with 4 output elements each (16-byte loads and stores), a
// work-group 256 / (HD/4) pairs; the partition loop is unrolled so several
// partials are in flight per thread.
template <int HD, int NF>
__global__ void __launch_bounds__(256)
attn_merge_kernel(const float *__restrict__ part_o, const float *__restrict__ part_ml,
                  const int32_t *__restrict__ lens, float *__restrict__ out, int n_heads,
                  int part_tokens, int split, int max_parts, int64_t max_len,
                  const int32_t *__restrict__ pre_parts, const float *__restrict__ pre_o,
                  const float *__restrict__ pre_ml, int max_pre_parts,
                  const int32_t *__restrict__ qmap, int64_t n_pairs, int folded) {
  constexpr int TPP = HD / 4;     // threads per (query, head)
  constexpr int PPW = 256 / TPP;  // pairs per work-group
  const int64_t pair = (int64_t)blockIdx.x * PPW + threadIdx.x / TPP;
  if (pair >= n_pairs) return;
  const int d = (threadIdx.x % TPP) * 4;
  const int h = (int)(pair % n_heads);
  const int64_t qx = pair / n_heads;
  const int64_t qi = qmap ? qmap[qx] : qx;
  const int64_t qh = qi * n_heads + h;
  const float *ml = part_ml + qh * max_parts * 2;
  // The first NF partials are loaded before the length is known (slots
  // clamped to max_parts - 1; slots past the query's np are never used, by
  // selection, so stale values there cannot leak), so the common case costs
  // one round trip.
  float m4[NF], l4[NF];
  f32x4 o4[NF];
#pragma unroll
  for (int p = 0; p < NF; ++p) {
    const int pc = p < max_parts ? p : max_parts - 1;
    m4[p] = ml[2 * pc];
    l4[p] = ml[2 * pc + 1];
    o4[p] = *reinterpret_cast<const f32x4 *>(part_o + (qh * max_parts + pc) * HD + d);
  }
  int64_t len = lens[qi];
  if (len < 0) len = 0;
  if (len > max_len) len = max_len;
  const int pt = split_partition(len, part_tokens, split);
  const int npre = pre_parts ? pre_parts[qi] : 0;
  if (npre < 0) return;  // its group wrote the output
  // A single partition wrote its output directly; with group partials too
  // when the context kernel folds them (`folded`), else it wrote a partial.
  // An empty remainder (np == 0) leaves the group partials to this kernel.
  const int np = div_up_tokens(len, pt);
  if (np <= 1 && npre == 0) return;
  if (np == 1 && folded) return;
  if (npre == 0 && np <= NF) {
    // The common case (a query of up to NF partitions, np <= max_parts).
    float mx = m4[0];
#pragma unroll
    for (int p = 1; p < NF; ++p) mx = p < np ? __builtin_fmaxf(mx, m4[p]) : mx;
    const float mref = mx == -INFINITY ? 0.f : mx;
    float lsum = 0.f;
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < NF; ++p) {
      if (p < np) {
        const float a = __builtin_amdgcn_exp2f(m4[p] - mref);
        lsum += l4[p] * a;
        o += o4[p] * a;
      }
    }
    f32x4 r = {0.f, 0.f, 0.f, 0.f};
    if (lsum > 0.f) r = f32x4{o.x / lsum, o.y / lsum, o.z / lsum, o.w / lsum};
    *reinterpret_cast<f32x4 *>(out + qh * HD + d) = r;
    return;
  }
  const float *pml = npre > 0 ? pre_ml + qh * max_pre_parts * 2 : nullptr;
  float mx = -INFINITY;
  for (int p = 0; p < np; ++p) mx = __builtin_fmaxf(mx, ml[2 * p]);
  for (int p = 0; p < npre; ++p) mx = __builtin_fmaxf(mx, pml[2 * p]);
  const float mref = mx == -INFINITY ? 0.f : mx;
  float lsum = 0.f;
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int p = 0; p < npre; ++p) {
    const float a = __builtin_amdgcn_exp2f(pml[2 * p] - mref);
    lsum += pml[2 * p + 1] * a;
    o += *reinterpret_cast<const f32x4 *>(pre_o + (qh * max_pre_parts + p) * HD + d) * a;
  }
#pragma unroll 4
  for (int p = 0; p < np; ++p) {
    const float a = __builtin_amdgcn_exp2f(ml[2 * p] - mref);
    lsum += ml[2 * p + 1] * a;
    o += *reinterpret_cast<const f32x4 *>(part_o + (qh * max_parts + p) * HD + d) * a;
  }
  f32x4 r = {0.f, 0.f, 0.f, 0.f};
  if (lsum > 0.f) r = f32x4{o.x / lsum, o.y / lsum, o.z / lsum, o.w / lsum};
  *reinterpret_cast<f32x4 *>(out + qh * HD + d) = r;
}

// Launch check of the attention kernel, then the partition merge when some
// query may span several partitions.
template <int HD>
hipError_t launch_merge(const AttnArgs &a, hipStream_t s, bool folded) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || (a.max_parts == 1 && !a.pre_parts) || (folded && a.merge_free)) return e;
  const int64_t pairs = a.n * a.n_heads;
  constexpr int ppw = 256 / (HD / 4);
  const unsigned mgrid = (unsigned)((pairs + ppw - 1) / ppw);
  // One round of loads for queries of up to four (eight) partitions.
  auto kern = a.max_parts <= 4 ? attn_merge_kernel<HD, 4> : attn_merge_kernel<HD, 8>;
  kern<<<mgrid, 256, 0, s>>>(a.part_o, a.part_ml, a.lens, a.out, a.n_heads, a.part_tokens, a.split, a.max_parts,
                             a.max_len, a.pre_parts, a.pre_o, a.pre_ml, a.max_pre_parts, a.qmap, pairs,
                             folded ? 1 : 0);
  return hipGetLastError();
}

// ----------------------------------------------------------------------------
// Kernel 4, 16-lane VALU form (f32 head_dim 64: one 16-byte load per lane
// covers a row across 16 lanes, a DPP row).
//
// Differences from attn_kernel, all aimed at VALU count per KV byte:
//  * the rows x heads partial dots of a tile are reduce-scattered over the 16
//    lanes of the row, so each lane ends with distinct scores instead of every
//    lane holding all of them. The head bits of the score index are split
//    with plain v[r] += dpp(v[r + n/2]) exchanges, with no per-lane selects,
//    because each lane's q registers are permuted once so that every DPP
//    partner map (mirror, half-mirror) flips exactly the head bit being
//    split; the two row bits take select steps, so K and V rows keep their
//    natural, coalesced lane order;
//  * the online softmax is distributed accordingly: each lane owns one head's
//    (max, sum) for its row group and evaluates one exp2 per score it holds;
//    the V pass fetches the weights it needs with row_newbcast;
//  * the accumulators are rescaled only when some running max grew (a
//    wave-uniform branch), which after the first tiles is rare;
//  * loads go through per-tile buffer descriptors (scalar) with 32-bit
//    per-lane offsets fixed for the whole loop; rows past the context and
//    prefetches past a wave's last tile fall outside the descriptor's extent
//    and read zeros without memory traffic, so the 2- or 3-stage tile
//    pipeline has no conditional loads.
// ----------------------------------------------------------------------------
// The four DPP partner maps of the scatter: lane ^ 15, ^ 7, ^ 2, ^ 1.
template <int T>
__device__ __forceinline__ float partner16(float x) {
  if constexpr (T == 0) return dpp<0x140>(x);       // row_mirror: lane ^ 15
  else if constexpr (T == 1) return dpp<0x141>(x);  // row_half_mirror: lane ^ 7
  else if constexpr (T == 2) return dpp<0x4E>(x);   // quad_perm [2,3,0,1]: lane ^ 2
  else return dpp<0xB1>(x);                         // quad_perm [1,0,3,2]: lane ^ 1
}

template <int K>
__device__ __forceinline__ float bcast16(float x) {
  // row_newbcast:K, lane K of each 16-lane row (every lane is written).
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x150 + K, 0xf, 0xf, false));
}

// The score layout of one scatter pass: N <= 16 partial dots per lane,
// index h * 2^RB + j (head h, row j of the pass). The scatter splits index
// bits from the top; head bits are split select-free (lane i keeps index
// r ^ g(i) in register r, g linear over GF(2) with g(lane ^ mask_t) =
// g(lane) ^ split_t, realised by permuting the lane's q registers), row bits
// with selects, so K rows stay in natural (coalesced) lane order.
template <int N, int RB>
struct Scatter16 {
  static_assert(N <= 16, "one score per lane at most");
  static constexpr int T = N == 16 ? 4 : (N == 8 ? 3 : (N == 4 ? 2 : 1));  // scatter steps
  static constexpr int half(int t) { return (N >> t) / 2; }  // index value of the bit split at t
  static constexpr bool free_step(int t) { return t < T && half(t) >= (1 << RB); }  // head bit
  static constexpr int gm(int t) { return free_step(t) ? half(t) : 0; }
  // g on the lane-bit basis e0..e3 (the masks 1, 2, 7, 15 span GF(2)^4).
  static constexpr int col(int b) {
    return b == 0 ? gm(3) : b == 1 ? gm(2) : b == 2 ? (gm(1) ^ gm(3) ^ gm(2)) : (gm(0) ^ gm(1));
  }
  static constexpr int lane_bit(int t) { return 8 >> t; }  // lane bit told apart by partner map t
  // Score index held by lane `lane` after the scatter.
  static constexpr int held(int lane) {
    int idx = 0;
    for (int b = 0; b < 4; ++b)
      if ((lane >> b) & 1) idx ^= col(b);
    for (int t = 0; t < T; ++t)
      if (!free_step(t) && (lane & lane_bit(t))) idx += half(t);
    return idx;
  }
  // A lane of the row holding score index idx.
  static constexpr int src(int idx) {
    for (int i = 0; i < 16; ++i)
      if (held(i) == idx) return i;
    return 0;
  }
};

// In-place reduce-scatter over the 16 lanes of a row; afterwards v[0]
// holds the row-wide sum of index held(lane).
template <int N, int RB, int n, int t>
__device__ __forceinline__ void reduce_scatter16(float (&v)[N], int lane) {
  using S = Scatter16<N, RB>;
  if constexpr (t < 4) {
    if constexpr (S::free_step(t)) {
#pragma unroll
      for (int r = 0; r < n / 2; ++r) v[r] += partner16<t>(v[r + n / 2]);
      reduce_scatter16<N, RB, n / 2, t + 1>(v, lane);
    } else if constexpr (t < S::T) {
      const bool up = (lane & S::lane_bit(t)) != 0;
#pragma unroll
      for (int r = 0; r < n / 2; ++r) {
        const float send = up ? v[r] : v[r + n / 2];
        const float keep = up ? v[r + n / 2] : v[r];
        v[r] = keep + partner16<t>(send);
      }
      reduce_scatter16<N, RB, n / 2, t + 1>(v, lane);
    } else {
      v[0] += partner16<t>(v[0]);
      reduce_scatter16<N, RB, n, t + 1>(v, lane);
    }
  }
}

// Max or sum over aligned groups of LANES lanes; steps below SKIP (lanes
// holding replicas of one value) are left out of a sum.
template <int LANES, int SKIP, bool MAX>
__device__ __forceinline__ float head_reduce(float x) {
  auto op = [](float a, float b) { return MAX ? __builtin_fmaxf(a, b) : a + b; };
  if constexpr (LANES > 1 && SKIP <= 1) x = op(x, dpp<0xB1>(x));
  if constexpr (LANES > 2 && SKIP <= 2) x = op(x, dpp<0x4E>(x));
  if constexpr (LANES > 4 && SKIP <= 4) x = op(x, dpp<0x141>(x));
  if constexpr (LANES > 8 && SKIP <= 8) x = op(x, dpp<0x140>(x));
  return x;
}

template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

template <typename T, int HD, int G, int NW>
__global__ void __launch_bounds__(64 * NW)
attn16_kernel(const T *__restrict__ kpool, const T *__restrict__ vpool, const float *__restrict__ q,
              const int32_t *__restrict__ tables, int64_t table_stride,
              const int32_t *__restrict__ lens, float *__restrict__ out, float *__restrict__ part_o,
              float *__restrict__ part_ml, int n_kv_heads, int64_t n_blocks, int64_t block_stride,
              int64_t slot_stride, int64_t head_stride, float qscale, int part_tokens,
              int max_parts, const int32_t *__restrict__ pre_parts,
              const int32_t *__restrict__ qmap, const int32_t *__restrict__ rows, int64_t n_rows,
            int64_t max_len, int32_t *__restrict__ status) {
  constexpr int E = Tile<T>::E;
  static_assert(HD / E == 16, "16 lanes per row");
  constexpr int RPL = 4, LOADS = 4;                             // rows per wave load, loads per tile
  constexpr int GP = G <= 1 ? 1 : G <= 2 ? 2 : G <= 4 ? 4 : 8;  // group padded to a power of two
  // Groups of 8 heads scatter the tile in two passes of two row slots, which
  // keeps 16 (not 32) partial dots live per lane.
  constexpr int PASSES = GP == 8 ? 2 : 1;
  constexpr int RPP = LOADS / PASSES;                 // row slots per pass
  constexpr int RB = RPP == 4 ? 2 : 1;                // log2(RPP)
  constexpr int N = GP * RPP;                         // partial dots per lane per pass (<= 16)
  using S = Scatter16<N, RB>;
  constexpr int NPL = PASSES;                         // scores per lane per tile
  constexpr int R = N < 16 ? 16 / N : 1;              // lanes holding the same score
  constexpr int LPH = 16 / GP;                        // lanes per head

  const int kvh = (int)(blockIdx.x % n_kv_heads);
  const int part = (int)((blockIdx.x / n_kv_heads) % max_parts);
  const int64_t qx = blockIdx.x / ((unsigned)n_kv_heads * max_parts);
  const int64_t qi = qmap ? qmap[qx] : qx;
  const int lane = threadIdx.x & 63;
  const int wave = NW == 1 ? 0 : __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, rg = lane >> 4;
  const int n_heads = n_kv_heads * G;

  int64_t len = lens[qi];
  if (len < 0) len = 0;
  if (len > max_len) len = max_len;
  // A query with group partials and nothing else to read (or whose group
  // wrote its output) has no work here.
  if (pre_parts && (pre_parts[qi] < 0 || (pre_parts[qi] > 0 && len == 0))) return;
  const int pt = partition_tokens(len, part_tokens);
  const int np = len > 0 ? (int)((len + pt - 1) / pt) : 1;
  if (part >= np) return;  // uniform over the work-group
  const int64_t tok0 = (int64_t)part * pt;
  const int64_t tok1 = len < tok0 + pt ? len : tok0 + pt;
  const int b0 = (int)(tok0 >> 4), b1 = (int)((tok1 + 15) >> 4);

  // Lane permutation of the head bits: register r of a pass's partial dots
  // holds head (r >> RB) ^ (gl >> RB), row r % RPP, so q slot u holds head
  // u ^ (gl >> RB). Heads past G are zero queries (padding).
  int gl = 0;
#pragma unroll
  for (int bit = 0; bit < 4; ++bit)
    if ((c >> bit) & 1) gl ^= S::col(bit);

  // Eight-head groups keep q in LDS (shared by the four waves and the four
  // row groups, read per head right before use); smaller groups keep it in
  // registers.
  constexpr bool kQInLds = GP == 8;
  __shared__ f32x4 sm_q[kQInLds ? GP * 16 * (E / 4) : 1];  // [slot u][lane c][E/4]
  float qv[kQInLds ? 1 : GP][E];
  {
    const float *qp = q + qi * (int64_t)n_heads * HD + (int64_t)kvh * G * HD + c * E;
    if constexpr (kQInLds) {
      if (threadIdx.x < 16) {
#pragma unroll
        for (int u = 0; u < GP; ++u) {
          const int h = u ^ (gl >> RB);
#pragma unroll
          for (int e = 0; e < E; e += 4) {
            f32x4 t = {0.f, 0.f, 0.f, 0.f};
            if (h < G) t = *reinterpret_cast<const f32x4 *>(qp + h * HD + e);
            sm_q[(u * 16 + c) * (E / 4) + e / 4] = t * qscale;
          }
        }
      }
      __syncthreads();
    } else {
#pragma unroll
      for (int u = 0; u < GP; ++u) {
        const int h = u ^ (gl >> RB);
#pragma unroll
        for (int e = 0; e < E; e += 4) {
          f32x4 t = {0.f, 0.f, 0.f, 0.f};
          if (h < G) t = *reinterpret_cast<const f32x4 *>(qp + h * HD + e);
#pragma unroll
          for (int i = 0; i < 4; ++i) qv[u][e + i] = t[i] * qscale;
        }
      }
    }
  }

  // Per-lane byte offsets inside a head tile, fixed for the whole loop.
  const uint32_t row_bytes = (uint32_t)(slot_stride * (int64_t)sizeof(T));
  const uint32_t col_off = (uint32_t)(c * 16);
  uint32_t roff[LOADS];
#pragma unroll
  for (int j = 0; j < LOADS; ++j) roff[j] = (uint32_t)(rg + RPL * j) * row_bytes + col_off;
  int my_row[NPL];  // tile rows of this lane's scores after the scatter
  {
    int jj = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (c == i) jj = S::held(i) & (RPP - 1);
#pragma unroll
    for (int pass = 0; pass < NPL; ++pass) my_row[pass] = rg + RPL * (pass * RPP + jj);
  }
  const char *kbase = reinterpret_cast<const char *>(kpool + (int64_t)kvh * head_stride);
  const char *vbase = reinterpret_cast<const char *>(vpool + (int64_t)kvh * head_stride);
  const int64_t block_bytes = block_stride * (int64_t)sizeof(T);

  float m_own = -INFINITY, l_own = 0.f;  // softmax state of this lane's head, row group rg
  float acc[G][E];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int e = 0; e < E; ++e) acc[h][e] = 0.f;

  const int32_t *tab = table_of(tables, table_stride, rows, n_rows, qi);
  check_table(tab, b0, b1, n_blocks, rows, n_rows, qi, status);

  // A tile is read through buffer descriptors whose extent ends at the last
  // row inside the context: rows past it (and every row of a prefetch past
  // the wave's last tile, extent 0) read as zeros without touching memory,
  // so every load is unconditional and the wait counts stay static.
  auto load_tile = [&](int b, u32x4 (&kr)[LOADS], u32x4 (&vr)[LOADS]) {
    const int bb = b < b1 ? b : b1 - 1;
    int32_t blk = tab[bb];
    if (blk < 0 || blk >= n_blocks) blk = 0;  // out-of-range entries read block 0 (never faults)
    const int valid = b < b1 ? (int)(tok1 - (int64_t)b * 16) : 0;
    const int rows = valid < 16 ? valid : 16;
    const int extent = rows > 0 ? (rows - 1) * (int)row_bytes + HD * (int)sizeof(T) : 0;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(kbase + (int64_t)blk * block_bytes), (short)0, extent, kBufferWord3);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(vbase + (int64_t)blk * block_bytes), (short)0, extent, kBufferWord3);
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
      kr[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, roff[j], 0, kNt));
      vr[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, roff[j], 0, kNt));
    }
  };

  auto compute_tile = [&](int b, const u32x4 (&kr)[LOADS], const u32x4 (&vr)[LOADS]) {
    const int valid = (int)(tok1 - (int64_t)b * 16);  // rows of this tile inside the context
    float sc[NPL];  // this lane's scores: one per pass
#pragma unroll
    for (int pass = 0; pass < PASSES; ++pass) {
      float v[N];
      // Keeps the LDS reads of q inside the loop (not hoisted into registers).
      if constexpr (kQInLds) asm volatile("" ::: "memory");
      float kf[RPP][E];
#pragma unroll
      for (int jj = 0; jj < RPP; ++jj) Tile<T>::unpack(kr[pass * RPP + jj], kf[jj]);
#pragma unroll
      for (int u = 0; u < GP; ++u) {
        float qu[E];
        if constexpr (kQInLds) {
#pragma unroll
          for (int e = 0; e < E; e += 4) {
            const f32x4 t = sm_q[(u * 16 + c) * (E / 4) + e / 4];
#pragma unroll
            for (int i = 0; i < 4; ++i) qu[e + i] = t[i];
          }
        } else {
#pragma unroll
          for (int e = 0; e < E; ++e) qu[e] = qv[u][e];
        }
#pragma unroll
        for (int jj = 0; jj < RPP; ++jj) {
          float a = 0.f;
#pragma unroll
          for (int e = 0; e < E; ++e) a = __builtin_fmaf(qu[e], kf[jj][e], a);
          v[u * RPP + jj] = a;
        }
      }
      reduce_scatter16<N, RB, N, 0>(v, lane);
      sc[pass] = v[0];
    }
    if (valid < 16) {
#pragma unroll
      for (int k = 0; k < NPL; ++k)
        if (my_row[k] >= valid) sc[k] = -INFINITY;
    }
    // Online softmax of this lane's head over the tile's rows of this row group.
    float bm = sc[0];
#pragma unroll
    for (int k = 1; k < NPL; ++k) bm = __builtin_fmaxf(bm, sc[k]);
    bm = head_reduce<LPH, 1, true>(bm);
    const float mn = __builtin_fmaxf(m_own, bm);
    const float mref = mn == -INFINITY ? 0.f : mn;
    const float alpha = __builtin_amdgcn_exp2f(m_own - mref);
    float p[NPL];
    float ps = 0.f;
#pragma unroll
    for (int k = 0; k < NPL; ++k) {
      p[k] = __builtin_amdgcn_exp2f(sc[k] - mref);
      ps += p[k];
    }
    ps = head_reduce<LPH, R, false>(ps);
    l_own = l_own * alpha + ps;
    const bool grew = mn > m_own;
    m_own = mn;
    if (__builtin_amdgcn_ballot_w64(grew)) {  // wave-uniform: some head's max grew
      static_for<0, G>([&](auto hc) {
        constexpr int h = decltype(hc)::value;
        const float a = bcast16<S::src(h * RPP)>(alpha);
#pragma unroll
        for (int e = 0; e < E; ++e) acc[h][e] *= a;
      });
    }
    static_for<0, LOADS>([&](auto jc) {
      constexpr int j = decltype(jc)::value;
      float vf[E];
      Tile<T>::unpack(vr[j], vf);
      static_for<0, G>([&](auto hc) {
        constexpr int h = decltype(hc)::value;
        // (head h, row slot j): pass j / RPP, index h * RPP + j % RPP of it
        const float w = bcast16<S::src(h * RPP + j % RPP)>(p[j / RPP]);
#pragma unroll
        for (int e = 0; e < E; ++e) acc[h][e] = __builtin_fmaf(w, vf[e], acc[h][e]);
      });
    });
  };

  // Software pipeline, STAGES - 1 tiles in flight while one is computed.
  // Loads past the wave's last tile read nothing (extent 0).
  constexpr int STAGES = GP <= 4 ? 3 : 2;
  {
    constexpr int W = NW;
    int b = b0 + wave;
    if (b < b1) {
      if constexpr (STAGES == 3) {
        u32x4 k0[LOADS], v0[LOADS], k1[LOADS], v1[LOADS], k2[LOADS], v2[LOADS];
        load_tile(b, k0, v0);
        load_tile(b + W, k1, v1);
        for (;;) {
          load_tile(b + 2 * W, k2, v2);
          compute_tile(b, k0, v0);
          if ((b += W) >= b1) break;
          load_tile(b + 2 * W, k0, v0);
          compute_tile(b, k1, v1);
          if ((b += W) >= b1) break;
          load_tile(b + 2 * W, k1, v1);
          compute_tile(b, k2, v2);
          if ((b += W) >= b1) break;
        }
      } else {
        u32x4 k0[LOADS], v0[LOADS], k1[LOADS], v1[LOADS];
        load_tile(b, k0, v0);
        for (;;) {
          load_tile(b + W, k1, v1);
          compute_tile(b, k0, v0);
          if ((b += W) >= b1) break;
          load_tile(b + W, k0, v0);
          compute_tile(b, k1, v1);
          if ((b += W) >= b1) break;
        }
      }
    }
  }

  // Every lane takes the (max, sum) of all heads of its row group, then the
  // four row groups of the wave are merged (lanes 16 and 32 apart).
  float m[G], l[G];
  static_for<0, G>([&](auto hc) {
    constexpr int h = decltype(hc)::value;
    m[h] = bcast16<S::src(h * RPP)>(m_own);
    l[h] = bcast16<S::src(h * RPP)>(l_own);
  });
#pragma unroll
  for (int off = 16; off < 64; off <<= 1) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float mo = __shfl_xor(m[h], off);
      const float lo = __shfl_xor(l[h], off);
      const float mn = __builtin_fmaxf(m[h], mo);
      const float mref = mn == -INFINITY ? 0.f : mn;
      const float as = __builtin_amdgcn_exp2f(m[h] - mref);
      const float ao = __builtin_amdgcn_exp2f(mo - mref);
      l[h] = l[h] * as + lo * ao;
#pragma unroll
      for (int e = 0; e < E; ++e) acc[h][e] = acc[h][e] * as + __shfl_xor(acc[h][e], off) * ao;
      m[h] = mn;
    }
  }

  const int64_t qh0 = qi * n_heads + (int64_t)kvh * G;
  const bool direct = np == 1 && !(pre_parts && pre_parts[qi] > 0);  // else merged later
  if constexpr (NW == 1) {
    // One wave: the lanes of row group 0 hold the merged numerators.
    if (rg == 0) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        if (direct) {
          const float inv = l[h] > 0.f ? 1.f / l[h] : 0.f;
          float *o = out + (qh0 + h) * HD + c * E;
#pragma unroll
          for (int e = 0; e < E; ++e) o[e] = l[h] > 0.f ? acc[h][e] * inv : 0.f;
        } else {
          const int64_t pi = (qh0 + h) * max_parts + part;
#pragma unroll
          for (int e = 0; e < E; ++e) part_o[pi * HD + c * E + e] = acc[h][e];
          if (c == 0) {
            part_ml[2 * pi] = m[h];
            part_ml[2 * pi + 1] = l[h];
          }
        }
      }
    }
    return;
  }

  // Merge the waves through LDS.
  __shared__ float sm_acc[NW][G][HD];
  __shared__ float sm_m[NW][G], sm_l[NW][G];
  if (rg == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
#pragma unroll
      for (int e = 0; e < E; ++e) sm_acc[wave][h][c * E + e] = acc[h][e];
      if (c == 0) {
        sm_m[wave][h] = m[h];
        sm_l[wave][h] = l[h];
      }
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < G * HD; idx += 64 * NW) {
    const int h = idx / HD, d = idx - h * HD;
    float mx = sm_m[0][h];
#pragma unroll
    for (int w = 1; w < NW; ++w) mx = __builtin_fmaxf(mx, sm_m[w][h]);
    const float mref = mx == -INFINITY ? 0.f : mx;
    float lsum = 0.f, o = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float a = __builtin_amdgcn_exp2f(sm_m[w][h] - mref);
      lsum += sm_l[w][h] * a;
      o += sm_acc[w][h][d] * a;
    }
    if (direct) {
      out[(qh0 + h) * HD + d] = lsum > 0.f ? o / lsum : 0.f;
    } else {
      const int64_t pi = (qh0 + h) * max_parts + part;
      part_o[pi * HD + d] = o;
      if (d == 0) {
        part_ml[2 * pi] = mx;
        part_ml[2 * pi + 1] = lsum;
      }
    }
  }
}

// ----------------------------------------------------------------------------
// Kernel 4 on the matrix cores (f16 and q8_0 tiles). In the VALU kernels
// every K element costs a G-way dot product and every V element a G-way
// FMA; with 1-byte q8_0 elements (or G > 4) that keeps the VALU busy for
// longer than the tile's bytes take to arrive. Here both products of a
// 16-token tile run on MFMA, one wave per (query, NH adjacent kv heads,
// partition), four waves to a work-group (kDecodeWaves); NH = 2 when the
// 2 G query heads fit the 16 columns (G <= 4),
// so each row segment read is two heads wide (512 B for f16), and each
// product then runs once per kv head, its Q' / P' zero outside that head's
// columns:
//   S^T[token][col] = K Q'^T   v_mfma_f32_16x16x32_f16, A = the K tile
//                              (staged through LDS into the A layout),
//                              B = Q' in registers;
//   O^T[d][col]   += V^T P'^T  v_mfma_f32_16x16x16_f16, A = V^T read from
//                              LDS with ds_read_b64_tr_b16, B = P' in the
//                              D layout of S^T (lane: tokens 4 (l/16) + j).
// Q' and P' hold f32 values as f16 hi + lo parts in mirrored columns (head
// h in column h, its lo part in column 15 - h): one MFMA covers both and a
// row_mirror DPP add joins them, so scores and sums keep f32 accuracy over
// exact f16 (or int8) elements. q8_0 tiles convert exactly to f16; each
// 32-element scale group is a k step of the score product, scaled after
// it, and a separate P' (P times the V group scale) for the O tiles of the
// group. The softmax reference per column is common to the four lane rows
// and raised only when a score exceeds it by kDecodeSlack (ballot), so the
// weights p = 2^(s - ref) <= 2^8 need no exchange on the fast path.
// ----------------------------------------------------------------------------
template <int B>
struct BufVec;
template <>
struct BufVec<16> {
  using type = u32x4;
  template <int AUX>
  __device__ static __forceinline__ type load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX));
  }
};
template <>
struct BufVec<8> {
  using type = u32x2;
  template <int AUX>
  __device__ static __forceinline__ type load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, AUX));
  }
};
template <>
struct BufVec<4> {
  using type = uint32_t;
  template <int AUX>
  __device__ static __forceinline__ type load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, AUX);
  }
};

// Stored quants x 8 (bytes u = x + 128) -> f16 x 8 of x, exact: each byte
// becomes the mantissa of an f16 in [1024, 1280) (bits 0x6400 | u, value
// 1024 + u), and 1152 is subtracted: two v_perm_b32 and two packed f16
// subtractions per four elements.
__device__ __forceinline__ h8 i8x8_to_h8(const u32x2 &w) {
  constexpr uint32_t kHi = 0x64646464u;
  const uint32_t a = w.x, b = w.y;
  const h2 bias = {(_Float16)1152.f, (_Float16)1152.f};
  const h2 p0 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(kHi, a, 0x04010400u)) - bias;
  const h2 p1 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(kHi, a, 0x04030402u)) - bias;
  const h2 p2 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(kHi, b, 0x04010400u)) - bias;
  const h2 p3 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(kHi, b, 0x04030402u)) - bias;
  return h8{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
}

constexpr float kDecodeSlack = 8.f;  // log2 headroom of the softmax reference

// The matrix-core products take Q as f16 operands. A query head whose scaled
// Q (x = q * scale * log2 e) reaches the f16 range (|x| >= 65504) enters them
// as x * 2^-e, e the smallest exponent that brings its largest element below
// 2^15 (exact: a power of two), and its scores are taken times 2^e after the
// product, so the result is the f32 computation's wherever that is finite.
// Heads inside the range keep e = 0 (factor 1: bits unchanged). amax is the
// head's largest |x| (NaN elements are ignored; an infinite one keeps e = 0
// and its scores are infinite or NaN, as in f32).
__device__ __forceinline__ int q_range_exp(float amax) {
  if (!(amax >= 65504.f) || !(amax <= 3.40282347e38f)) return 0;
  return __builtin_amdgcn_frexp_expf(amax) - 15;
}

// ----------------------------------------------------------------------------
// Work order of the decode grid. The grid's items are (query, partition)
// pairs (times the kv-head groups, fastest). Taken in query order, a batch of
// mixed lengths leaves the SIMDs whose waves drew short partitions idle while
// the longest ones finish, and the chip stops being bandwidth-bound well
// before the end. So the items are taken by descending size class (32-token
// classes), then query index, then partition: the hardware hands
// work-groups to freed SIMDs in grid order, which makes this longest-first
// list scheduling. Each wave finds its item from the lengths alone (one
// histogram in LDS, one prefix scan per 64 queries), so nothing is computed
// or uploaded per step on the host; a query's partitions and result bits do
// not depend on where its items land.
//
// When the batch holds at least twice as many partitions (times the kv-head
// groups) as the chip holds waves at once, an item is a run of k consecutive
// partitions of one query, k = partitions / wave slots: one wave streams
// them back to back and writes each partition's partial as it passes its
// end, so every partial (and every output bit) is the one a wave per
// partition writes, while each wave pays its start (order scan, first table
// entries and loads: ~7 us) once per k partitions (32 queries x 32768
// tokens: 4096 partition items on 1024 slots, k = 4). Size classes then
// count 32 k tokens.
// ----------------------------------------------------------------------------
constexpr int kOrderClasses = 32;  // size classes of an item (32 k tokens each)
constexpr int kOrderMaxQueries = 256;  // beyond this, query order (the scans would cost more)
constexpr int kOrderChunks = kOrderMaxQueries / 64;

__device__ __forceinline__ int order_class(int tokens, int k) {
  const int c = (tokens / k) >> 5;
  return c < kOrderClasses - 1 ? c : kOrderClasses - 1;
}

// Query q's length (clamped), partition size and partition count.
__device__ __forceinline__ void decode_query_parts(const int32_t *__restrict__ lens, int64_t q, int64_t max_len,
                                                   int part_tokens, int split, int &clen, int &pt, int &np) {
  int64_t len = lens[q];
  if (len < 0) len = 0;
  if (len > max_len) len = max_len;
  clen = (int)len;
  pt = split_partition(len, part_tokens, split);
  np = len > 0 ? div_up_tokens(len, pt) : 1;
}

// Size classes and item counts of queries lane, 64 + lane, ... (n <=
// kOrderMaxQueries; zero past n), and the items per class in `hist`
// (kOrderClasses ints of LDS): a query's items are runs of k partitions, all
// but the last of k partitions (class key), the last of the tokens left
// (class keyl; 0 tokens for an empty query), so the list is longest first
// item by item. One wave; returns k (the same in every wave: it depends on
// the lengths, the grid's kv-head groups, the wave slots and max_run only).
struct OrderShapes {
  int key[kOrderChunks], keyl[kOrderChunks], items[kOrderChunks], len[kOrderChunks];
};

template <bool FIRST_WAVE_COUNTS = false, bool RUNS = false>
__device__ __forceinline__ int decode_order_setup(const int32_t *__restrict__ lens, int64_t n, int64_t max_len,
                                                  int part_tokens, int split, int lane, int32_t *hist,
                                                  OrderShapes &sh, int n_groups, int slots, int max_run) {
  if (lane < kOrderClasses) hist[lane] = 0;
  __syncthreads();
  int pt[kOrderChunks];
  int k = 1;
#pragma unroll
  for (int c = 0; c < kOrderChunks; ++c) {
    sh.key[c] = 0;
    sh.keyl[c] = 0;
    sh.items[c] = 0;
    sh.len[c] = 0;
    pt[c] = 1;
    if ((int64_t)c * 64 + lane < n)
      decode_query_parts(lens, (int64_t)c * 64 + lane, max_len, part_tokens, split, sh.len[c], pt[c],
                         sh.items[c]);
  }
  if constexpr (RUNS) {  // the run length from the batch's partition items (a wave-wide sum)
    int total = 0;
#pragma unroll
    for (int c = 0; c < kOrderChunks; ++c) total += sh.items[c];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) total += __shfl_xor(total, off);
    const int64_t waves = (int64_t)__builtin_amdgcn_readfirstlane(total) * n_groups;
    k = slots > 0 && waves >= 2 * (int64_t)slots ? (int)(waves / slots) : 1;
    k = k < max_run ? k : max_run;
  } else {
    (void)n_groups;
    (void)slots;
    (void)max_run;
  }
#pragma unroll
  for (int c = 0; c < kOrderChunks; ++c) {
    if ((int64_t)c * 64 + lane < n) {
      const int np = sh.items[c], len = sh.len[c];
      const int items = (np + k - 1) / k;
      sh.items[c] = items;
      sh.key[c] = order_class(k * pt[c], k);
      sh.keyl[c] = order_class(len > 0 ? len - (items - 1) * k * pt[c] : 0, k);
      // (several waves per work-group: every wave finds the shapes, the
      // first one counts them)
      if (!FIRST_WAVE_COUNTS || threadIdx.x < 64) {
        if (items > 1) atomicAdd(hist + sh.key[c], items - 1);  // LDS
        atomicAdd(hist + sh.keyl[c], 1);
      }
    }
  }
  __syncthreads();
  return k;
}

// Item t of the ordered list: its query qx and partition part, or false when
// t is past the last item. Every decision and result is uniform over the
// wave (read-first-lane of the exchanged values), so the item's addresses
// stay in scalar registers.
__device__ __forceinline__ bool decode_order_find(int64_t t, int64_t n, int lane, const int32_t *hist,
                                                  const OrderShapes &sh, int64_t &qx, int &part, int &qlen) {
  int cls = -1;
  int64_t base = 0;
  for (int k = kOrderClasses - 1; k >= 0; --k) {
    const int c = __builtin_amdgcn_readfirstlane(hist[k]);
    if (t < base + c) {
      cls = k;
      break;
    }
    base += c;
  }
  if (cls < 0) return false;
  t -= base;
#pragma unroll
  for (int c = 0; c < kOrderChunks; ++c) {
    const int64_t c0 = (int64_t)c * 64;
    if (c0 >= n) break;
    // this class's items of the lane's query: its full partitions (parts
    // 0 .. items - 2) and / or its last one (part items - 1)
    const int v = (sh.key[c] == cls ? sh.items[c] - 1 : 0) + (sh.keyl[c] == cls ? 1 : 0);
    int incl = v;  // inclusive prefix sum over the wave
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(incl, d, 64);
      if (lane >= d) incl += y;
    }
    const int tot = __builtin_amdgcn_readfirstlane(__shfl(incl, 63, 64));
    if (t < tot) {
      const uint64_t hit = __builtin_amdgcn_ballot_w64(incl > t);
      const int j = __builtin_ctzll(hit);
      const int end = __builtin_amdgcn_readfirstlane(__shfl(incl, j, 64));
      const int cnt = __builtin_amdgcn_readfirstlane(__shfl(v, j, 64));
      const int key = __builtin_amdgcn_readfirstlane(__shfl(sh.key[c], j, 64));
      const int items = __builtin_amdgcn_readfirstlane(__shfl(sh.items[c], j, 64));
      qlen = __builtin_amdgcn_readfirstlane(__shfl(sh.len[c], j, 64));
      qx = c0 + j;
      part = key == cls ? (int)(t - (end - cnt)) : items - 1;
      return true;
    }
    t -= tot;
  }
  return false;
}

// The weight operand's part for each lane: the lo part f16(x - f16(x)) on lo
// lanes, else the hi part f16(x) (columns past the group are discarded, any
// finite value does).
//
// q8_0 weights x = p d (d the token's V scale, f16): hi = f16(p d), then
// f16(p d + c) with c = hi * lo_m2 (lo_m2 = -1 on lo lanes, 0 on the others,
// one v_pk_mul_f16 per pair) is the lo part on lo lanes and hi on the others;
// p d is exact inside v_fma_mix, so the lo part is f16(p d - hi).
__device__ __forceinline__ h4 weight_parts_scaled(const float (&p)[4], const h4 &d, const h2 &lo_m2) {
  h4 r;
#pragma unroll
  for (int i = 0; i < 4; i += 2) {
    const h2 hi = h2{(_Float16)__builtin_fmaf(p[i], (float)d[i], 0.f),
                     (_Float16)__builtin_fmaf(p[i + 1], (float)d[i + 1], 0.f)};
    const h2 c = hi * lo_m2;
    r[i] = (_Float16)__builtin_fmaf(p[i], (float)d[i], (float)c[0]);
    r[i + 1] = (_Float16)__builtin_fmaf(p[i + 1], (float)d[i + 1], (float)c[1]);
  }
  return r;
}

// The parts of four f32 weights: lo_mult is -1 on lo lanes and 0 on the
// others, in a register, so f16(fma(f16(x), lo_mult, x)) is either part, one
// v_fma_mix on the packed hi parts per element.
__device__ __forceinline__ h4 weight_parts(const float (&x)[4], float lo_mult) {
  const h2 h01 = __builtin_convertvector(f32x2{x[0], x[1]}, h2);
  const h2 h23 = __builtin_convertvector(f32x2{x[2], x[3]}, h2);
  h4 r;
  r[0] = (_Float16)__builtin_fmaf((float)h01[0], lo_mult, x[0]);
  r[1] = (_Float16)__builtin_fmaf((float)h01[1], lo_mult, x[1]);
  r[2] = (_Float16)__builtin_fmaf((float)h23[0], lo_mult, x[2]);
  r[3] = (_Float16)__builtin_fmaf((float)h23[1], lo_mult, x[3]);
  return r;
}

// Stored quants x 8 -> f16 x 8 of 1152 + x (exact; the bias is taken out
// after the product, where it costs one subtraction per score instead of
// one per element).
__device__ __forceinline__ h8 i8x8_to_h8_biased(const u32x2 &w) {
  constexpr uint32_t kHi = 0x64646464u;
  const uint32_t a = w.x, b = w.y;
  const u32x4 r = {__builtin_amdgcn_perm(kHi, a, 0x04010400u), __builtin_amdgcn_perm(kHi, a, 0x04030402u),
                   __builtin_amdgcn_perm(kHi, b, 0x04010400u), __builtin_amdgcn_perm(kHi, b, 0x04030402u)};
  return __builtin_bit_cast(h8, r);
}

// Waves per work-group of the matrix-core decode kernel: four consecutive
// waves of the grid, i.e. the kv-head groups of one (query, partition) item
// on one CU, which then reads whole pool rows together (each wave still
// streams its own item; bit-identical results). Measured against one wave
// per work-group: the Llama-3-8B fused decode step 140.9 -> 137.9 us (the
// kernel ~134 us in the plain, graph and fused passes alike instead of
// 133-137), q8_0 decode 3.5% and the Qwen2.5-7B step 2% faster, 32 x 32k
// decode within the noise, config 3's per-query pass 1.4% slower. The wave
// index is made scalar (readfirstlane) and the grid index kept 32-bit: as a
// vector value or a 64-bit division it cost SGPR spills and 10%.
constexpr int kDecodeWaves = 4;

template <typename T, int HD, int G, int NH, bool RUNS>
__global__ void __launch_bounds__(64 * kDecodeWaves)
attn_mfma_kernel(const T *__restrict__ kpool, const T *__restrict__ vpool, const float *__restrict__ q,
                 const int32_t *__restrict__ tables, int64_t table_stride,
                 const int32_t *__restrict__ lens, float *__restrict__ out, float *__restrict__ part_o,
                 float *__restrict__ part_ml, int n_kv_heads, int64_t n_blocks, int64_t block_stride,
                 int64_t slot_stride, int64_t head_stride, float qscale, int part_tokens,
                 int split, int max_parts, const int32_t *__restrict__ pre_parts,
                 const int32_t *__restrict__ qmap, const uint16_t *__restrict__ kscale,
                 const uint16_t *__restrict__ vscale, const int32_t *__restrict__ rows, int64_t n_rows,
                 int64_t max_len, const float *__restrict__ pre_o, const float *__restrict__ pre_ml,
                 int max_pre_parts, const int32_t *__restrict__ new_slots,
                 const float *__restrict__ new_k, const float *__restrict__ new_v, int64_t new_stride,
                 T *kdst, T *vdst, int64_t n_queries, int order, int slots, int pair_items,
                 int32_t *__restrict__ status) {
#ifdef LTKV_TIMELINE
  unsigned long long tl_[8] = {__builtin_amdgcn_s_memrealtime(), 0, 0, 0, 0, 0, 0, 0};
#endif
  // Issue priority (s_setprio) among the waves of a SIMD: the highest until
  // the first tiles' loads are issued, then by tiles left (wave_priority).
  // Where two waves share a SIMD, the one that arrived first otherwise wins
  // nearly every vector-memory issue slot while the memory system is
  // saturated: a wave arriving beside a streaming one took ~15 us to issue
  // its first loads, and the first waves finished long before the second
  // ones (Qwen2.5-7B step, 120 queries: first waves done at ~89 us, second
  // ones at ~156 us, a tail of one wave per SIMD after them). Priorities
  // change nothing for correctness.
  __builtin_amdgcn_s_setprio(3);
  constexpr bool Q8 = std::is_same_v<T, int8_t>;
  constexpr int KS = HD / 32;              // score k steps: one q8_0 scale group each
  constexpr int DT = HD / 16;              // 16-row tiles of O^T
  constexpr int RB = HD * (int)sizeof(T);  // bytes of one head's row
  constexpr int HP = RB / 16;              // 16-byte pieces of a head row
  constexpr int LPR = NH * HP;             // lanes per row segment (NH adjacent heads)
  constexpr int RPI = 64 / LPR;            // rows per load instruction
  constexpr int NLD = 16 / RPI;            // load instructions per tile, K or V
  constexpr int KB = 8 * (int)sizeof(T);   // bytes of an A slice of the score product
  // LDS bytes per staged K row (as loaded) and V row (f16). f16 rows of 128
  // elements take 32 bytes of pad: SQ_LDS_BANK_CONFLICT per launch 3.2 M ->
  // 0.02 M at the Llama-3-8B shape (time unchanged) and 4.2 M -> 0.07 M at
  // the Qwen2.5-7B step (1% faster) against 16; q8_0 rows keep 16 (a K pad
  // of 32 gave more conflicts, 8.0 M -> 9.5 M, and 1% more time; a V pad
  // of 32 fewer, 6.4 M, at the same time).
  constexpr int KPITCH = RB + (!Q8 && HD == 128 ? 32 : 16);
  constexpr int VPITCH = HD * 2 + (!Q8 && HD == 128 ? 32 : 16);
  constexpr int NQ = NH * G;               // query heads of the wave
  constexpr int NSC = NH * KS * 16;        // q8_0 scale entries of a tile, K or V
  constexpr int STAGES = NH == 2 && Q8 ? 2 : 3;  // tiles in flight + 1
  using KV = typename BufVec<KB>::type;
  using SV = uint32_t;  // one or two b16 scale entries
  static_assert(NQ <= 8, "hi and lo columns of the wave's query heads must fit 16");
  static_assert(HD == 64 || HD == 128, "head_dim 64 or 128");
  static_assert(LPR <= 64 && RPI * NLD == 16, "row segment must split over the wave");
  constexpr int NW = kDecodeWaves;
  // the wave in its work-group (uniform: kept in a scalar register)
  const int wv = NW == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  __shared__ __attribute__((aligned(16))) char sk_w[NW][NH][16 * KPITCH];
  __shared__ __attribute__((aligned(16))) char sv_w[NW][NH][16 * VPITCH];
  __shared__ __attribute__((aligned(16))) uint16_t ssc_w[NW][2][Q8 ? NSC : 1];  // q8_0: K, V scales of a tile
  auto &sk = sk_w[wv];
  auto &sv = sv_w[wv];
  auto &ssc = ssc_w[wv];
  // RUNS (ordered launches with many more partitions than wave slots, f16
  // two-head waves): a wave may stream a run of up to kRunSlots + 1
  // partitions. The partials of a run's partitions before its last stay in
  // LDS until the wave's end: stores inside the tile loop make the waits for
  // the loads issued after them wait for the stores too (vector memory
  // operations complete in order), and under the loop's load traffic such a
  // store took ~19 us to complete (32 x 32768 tokens: 686 us with the
  // partials stored as they end, 630 us without the stores). The slots fit
  // beside the tiles at one work-group per CU. The run logic costs registers
  // and a scheduling boundary per tile, so launches that cannot form runs
  // take the kernel without it (RUNS false): kernels at two waves per SIMD
  // (q8_0, one-head waves) lost their occupancy or 3% with it.
  static_assert(!RUNS || (NH == 2 && !Q8), "runs of partitions: f16 two-head waves");
  constexpr int kRunSlots = RUNS ? 3 : 1;
  __shared__ __attribute__((aligned(16))) f32x4 srun_o[NW][kRunSlots][RUNS ? DT : 1][RUNS ? NQ * 4 : 1];
  __shared__ float srun_ml[NW][kRunSlots][RUNS ? NQ : 1][2];

  __shared__ int32_t shist[kOrderClasses];

  // 1-D grid of (wave, NH-head group), the head group fastest. Wave w of a
  // head group streams one item: without `order`, partition w % max_parts of
  // query w / max_parts; with `order`, item w of the longest-first list
  // (decode_order_find), a run of `run` consecutive partitions of a query.
  const int n_groups = n_kv_heads / NH;
  const unsigned gw = blockIdx.x * NW + wv;  // the grid's wave (the launch keeps it below 2^32)
  const int kvh0 = (int)(gw % n_groups) * NH;
  const int lane = threadIdx.x & 63;
  const int lr = lane & 15, lq = lane >> 4;
  const int n_heads = n_kv_heads * G;
  int64_t wave_idx = gw / n_groups;
  // Two work-groups per CU (pair_items > 0: the items of the chip's first
  // round of work-groups): the grid's first pair_items / 2 items and the
  // next ones share CUs, so the second half takes its items in reverse (the
  // longest item with the shortest of the round) and the pairs a CU's SIMDs
  // hold add up to about the same tiles (q8_0 decode 87.5 -> 85.7 us). The
  // reversal is a permutation of the grid's complete items [p / 2, p), so
  // every item of the list still has its wave.
  if (order && pair_items > 0) {
    const int64_t w_items = (int64_t)gridDim.x * NW / n_groups;
    const int64_t p = pair_items < w_items ? pair_items : w_items;
    if (wave_idx >= p / 2 && wave_idx < p) wave_idx = p / 2 + (p - 1 - wave_idx);
  }
  OrderShapes osh;
  int run = 1;
  if (order)
    run = decode_order_setup<(NW > 1), RUNS>(lens, n_queries, max_len, part_tokens, split, lane, shist, osh,
                                             n_groups, slots, kRunSlots + 1);

  // B operands Q'_a^T of the score product, one per kv head a of the wave:
  // column lr < NQ holds the hi part of query head lr of the wave, column
  // 15 - j the lo part of query head j; a column is nonzero only in the
  // operand of its query head's kv head (j / G).
  const bool hi_lane = lr < NQ, lo_lane = lr >= 16 - NQ;
  float lo_mult = lo_lane ? -1.f : 0.f;  // weight_parts: opaque to the optimiser
  asm volatile("" : "+v"(lo_mult));
  h2 lo_m2 = lo_lane ? h2{-1.f16, -1.f16} : h2{0.f16, 0.f16};  // weight_parts_scaled
  asm volatile("" : "+v"(lo_m2));
  const int qj = hi_lane ? lr : (lo_lane ? 15 - lr : 0);  // the column's query head in the wave
  const int my_head = qj / G;                             // its kv head in the wave
  // The query operand is fetched (fetch_q) and converted (convert_q) apart:
  // the conversion waits for the fetch, and the first tiles' loads are issued
  // in between, so the two latencies overlap. q8_0 K enters the score product
  // as 1152 + k: 1152 times the column's sum of each k step of Q' comes off
  // afterwards (qbias).
  auto fetch_q = [&](int64_t qi, f32x4 (&qr)[2 * KS]) __attribute__((always_inline)) {
    const float *qp = q + qi * (int64_t)n_heads * HD + ((int64_t)kvh0 * G + qj) * HD + 8 * lq;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qr[2 * ks] = *reinterpret_cast<const f32x4 *>(qp + 32 * ks);
      qr[2 * ks + 1] = *reinterpret_cast<const f32x4 *>(qp + 32 * ks + 4);
    }
  };
  // Heads beyond the f16 range (q_range_exp): the column's factor 2^e for
  // its scores, and whether any column of the wave has one (uniform).
  float qmul = 1.f;
  bool qscaled = false;
  auto convert_q = [&](const f32x4 (&qr)[2 * KS], h8 (&qb)[NH][KS], float (&qbias)[KS]) __attribute__((always_inline)) {
    float amax = 0.f;  // over the column's head: its 128 (64) elements lie in lanes lr + 16 lq
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e)
        amax = __builtin_fmaxf(amax, __builtin_fabsf((e < 4 ? qr[2 * ks][e] : qr[2 * ks + 1][e - 4]) * qscale));
    amax = __builtin_fmaxf(amax, __shfl_xor(amax, 16));
    amax = __builtin_fmaxf(amax, __shfl_xor(amax, 32));
    const int qex = q_range_exp(amax);
    const float qinv = __builtin_ldexpf(1.f, -qex);
    qmul = __builtin_ldexpf(1.f, qex);
    qscaled = __builtin_amdgcn_ballot_w64(qex != 0) != 0;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = (e < 4 ? qr[2 * ks][e] : qr[2 * ks + 1][e - 4]) * qscale * qinv;
        const _Float16 h = (_Float16)x;
        const _Float16 part_x = hi_lane ? h : (lo_lane ? (_Float16)(x - (float)h) : (_Float16)0.f);
#pragma unroll
        for (int a = 0; a < NH; ++a) qb[a][ks][e] = a == my_head ? part_x : (_Float16)0.f;
      }
    }
    if constexpr (Q8) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        float t = 0.f;
#pragma unroll
        for (int a = 0; a < NH; ++a)
#pragma unroll
          for (int e = 0; e < 8; ++e) t += (float)qb[a][ks][e];
        t += __shfl_xor(t, 16);
        t += __shfl_xor(t, 32);
        qbias[ks] = 1152.f * t;
      }
    }
  };

  // Loads: lane l takes 16-byte piece l % LPR of rows RPI i + l / LPR of the
  // wave's row segment (NH adjacent heads); piece p is head p / HP, bytes
  // 16 (p % HP) of its row.
  const int piece = lane % LPR, prow = lane / LPR;
  const int ph = piece / HP, pc = piece % HP;
  const uint32_t row_bytes = (uint32_t)(slot_stride * (int64_t)sizeof(T));
  uint32_t roff[NLD];
#pragma unroll
  for (int i = 0; i < NLD; ++i) roff[i] = (uint32_t)(RPI * i + prow) * row_bytes + (uint32_t)(piece * 16);
  // q8_0 scales: the wave's heads' groups of a block are one run [NH KS
  // groups][16 slots]; lane l loads entry l % NSC (or entries 2l, 2l + 1).
  const int64_t sgroups = slot_stride >> 5;
  const int64_t shead = ((int64_t)kvh0 * head_stride >> 5) * 32;
  const int sidx = NSC <= 64 ? lane % NSC : 2 * lane;
  const char *kbase = reinterpret_cast<const char *>(kpool + (int64_t)kvh0 * head_stride);
  const char *vbase = reinterpret_cast<const char *>(vpool + (int64_t)kvh0 * head_stride);
  const int64_t block_bytes = block_stride * (int64_t)sizeof(T);

  float m_ref = -INFINITY, l_run = 0.f;  // softmax reference and sum of this lane's column
  // Set with the reference: the raise threshold (m_ref + slack) and the
  // exponent offset (m_ref, 0 while there is none).
  float m_thr = -INFINITY, m_off = 0.f;
  // O^T accumulators. q8_0 pairs keep one set per kv head of the pair (the
  // lane's own head's set is taken at the end), so the weight operand needs
  // no per-head zeroing in every scale group; f16 pairs share one set (their
  // registers are full) and zero the other head's columns once per tile.
  constexpr int OS = Q8 ? NH : 1;
  f32x4 oacc[OS][DT];
  auto reset = [&]() __attribute__((always_inline)) {
    m_ref = -INFINITY;
    m_thr = -INFINITY;
    m_off = 0.f;
    l_run = 0.f;
#pragma unroll
    for (int a = 0; a < OS; ++a)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) oacc[a][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  };

  // One item: a partition [tok0, tok1) of query qi (tiles b0 .. b1 - 1).
  // Every field is uniform over the wave (scalar registers).
  struct Item {
    int64_t qi, len, tok1;
    int part, np, b0, b1;  // part: the partition of tile b (the item's first one at the start)
    int p0, plast, pt_tiles;  // the item's first and last partitions; tiles per partition
    const int32_t *tab;
    int b_new, r_new;  // fused new row: its tile and row (b_new -1: none)
    int32_t cell;      // ... and its pool cell
    bool valid;
  };
  // The wave's item (valid false: none), with its query operand (qr) and
  // fused new row (kr, vr) fetched, as f32.
  auto make_item = [&](Item &it, f32x4 (&qr)[2 * KS], f32x4 (&kr)[2], f32x4 (&vr)[2]) __attribute__((always_inline)) {
    it.valid = false;
    int64_t qx;
    int part, olen = 0;
    if (order) {
      if (!decode_order_find(wave_idx, n_queries, lane, shist, osh, qx, part, olen)) return;
      // uniform over the wave: keep them (and the table and buffer addresses
      // derived from them) in scalar registers
      qx = __builtin_amdgcn_readfirstlane((int)qx);
      part = __builtin_amdgcn_readfirstlane(part);
    } else {
      part = (int)(wave_idx % max_parts);
      qx = wave_idx / max_parts;
      if (NW > 1 && qx >= n_queries) return;  // waves past the grid's last item
    }
    const int64_t qi = qmap ? qmap[qx] : qx;
    int64_t len;
    if (order) {
      len = olen;  // the order scan read and clamped it (ordered launches have no query map)
    } else {
      len = lens[qi];
      if (len < 0) len = 0;
      if (len > max_len) len = max_len;
    }
    // A query with group partials and nothing else to read (or whose group
    // wrote its output) has no work here.
    if (pre_parts && (pre_parts[qi] < 0 || (pre_parts[qi] > 0 && len == 0))) return;
    const int pt = split_partition(len, part_tokens, split);
    const int np = len > 0 ? div_up_tokens(len, pt) : 1;
    // the item's partitions: run of them from part * run (run 1 without order)
    part *= run;
    if (part >= np) return;
    const int plast = part + run - 1 < np - 1 ? part + run - 1 : np - 1;
    const int64_t tok0 = (int64_t)part * pt, tend = (int64_t)(plast + 1) * pt;
    it.qi = qi;
    it.len = len;
    it.part = part;
    it.p0 = part;
    it.plast = plast;
    it.pt_tiles = pt >> 4;  // partitions are multiples of 32 tokens
    it.np = np;
    it.tok1 = len < tend ? len : tend;
    it.b0 = (int)(tok0 >> 4);
    it.b1 = (int)((it.tok1 + 15) >> 4);
    // A resident row outside the tables reads row 0 and is a fault when the
    // query has tokens (table entries are checked as their tiles load).
    int64_t trow = qi;
    if (rows) {
      trow = scalar_read(rows, qi);
      if (trow < 0 || trow >= n_rows) {
        if (it.b1 > it.b0) report_fault(status, kFaultTable, qi);
        trow = 0;
      }
    }
    it.tab = tables + trow * table_stride;
    fetch_q(qi, qr);

    // Fused append (f16, decode steps): the wave of the query's last partition
    // writes the query's new K/V row (position len - 1, cell new_slots[qi]) of
    // its heads, rounded to f16 as write_kernel does, and uses those registers
    // for that row of the last tile instead of loading it (commit_new). Every
    // lane takes the 16-byte piece it loads (lanes of different rows hold the
    // same piece and store the same bytes): no lane test, so the item's
    // fields stay uniform.
    it.b_new = -1;
    it.r_new = 0;
    it.cell = -1;
    kr[0] = kr[1] = vr[0] = vr[1] = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (!Q8) {
      if (new_slots && plast == np - 1 && len > 0) {  // uniform
        const int32_t cell = scalar_read(new_slots, qi);
        // The cell must be position len - 1 of the query's table (what the
        // claim returned for it); otherwise write-then-attend would differ.
        if (cell >= 0 && (int64_t)scalar_read(it.tab, (len - 1) >> 4) * 16 + ((len - 1) & 15) != (int64_t)cell)
          report_fault(status, kFaultFusedCell, qi);
        if (cell >= 0 && (int64_t)cell < n_blocks * 16) {
          it.b_new = (int)((len - 1) >> 4);
          it.r_new = (int)((len - 1) & 15);
          it.cell = cell;
          const float *ksrc = new_k + qi * new_stride + (int64_t)kvh0 * head_stride + 8 * piece;
          const float *vsrc = new_v + qi * new_stride + (int64_t)kvh0 * head_stride + 8 * piece;
          kr[0] = *reinterpret_cast<const f32x4 *>(ksrc);
          kr[1] = *reinterpret_cast<const f32x4 *>(ksrc + 4);
          vr[0] = *reinterpret_cast<const f32x4 *>(vsrc);
          vr[1] = *reinterpret_cast<const f32x4 *>(vsrc + 4);
        }
      }
    }
    it.valid = true;
  };

  // The item's fused row as f16 (nk, nv), written to its pool cell.
  auto commit_new = [&](const Item &it, const f32x4 (&kr)[2], const f32x4 (&vr)[2], u32x4 &nk, u32x4 &nv) __attribute__((always_inline)) {
    nk = u32x4{pack_f16x2(kr[0].x, kr[0].y), pack_f16x2(kr[0].z, kr[0].w), pack_f16x2(kr[1].x, kr[1].y),
               pack_f16x2(kr[1].z, kr[1].w)};
    nv = u32x4{pack_f16x2(vr[0].x, vr[0].y), pack_f16x2(vr[0].z, vr[0].w), pack_f16x2(vr[1].x, vr[1].y),
               pack_f16x2(vr[1].z, vr[1].w)};
    if constexpr (!Q8) {
      if (it.cell >= 0) {  // uniform
        const int64_t dst = (int64_t)it.cell * slot_stride + (int64_t)kvh0 * head_stride + 8 * piece;
        *reinterpret_cast<u32x4 *>(kdst + dst) = nk;
        *reinterpret_cast<u32x4 *>(vdst + dst) = nv;
      }
    }
  };

  struct Stage {
    u32x4 k[NLD], v[NLD];
    SV ks, vs;  // q8_0: scale entries sidx (.. sidx + 1) of K and of V
  };

  // The wave's item, its query operand (qb, qbias) and fused row (nk, nv).
  Item cur;
  h8 qb[NH][KS];
  float qbias[KS];
  u32x4 nk, nv;

  // Loads go through buffer descriptors whose extent ends at the last row
  // inside the context: rows past it, and every row of a load past the last
  // tile (live false), read as zeros without touching memory.
  // A table entry outside the pool reads block 0 instead (never faults); the
  // query of the last one is reported when the wave ends (a store inside the
  // tile loop would keep the compiler from reading the tables through the
  // scalar cache).
  int64_t fault_q = -1;
  auto load_tile = [&](int32_t entry, int64_t qi, int64_t tok1, int b_new, int r_new, bool live, int b,
                       Stage &st) __attribute__((always_inline)) {
    int32_t blk = 0;
    int rows = 0, lrows = 0;
    if (live) {  // uniform; b is a tile of the item, in [b0, b1); entry is its table entry
      blk = entry;
      const bool bad = blk < 0 || blk >= n_blocks;
      fault_q = bad ? qi : fault_q;
      blk = bad ? 0 : blk;
      const int valid = (int)(tok1 - (int64_t)b * 16);
      rows = valid < 16 ? valid : 16;
      // the fused new row (the tile's last valid row) is not loaded
      lrows = b == b_new ? r_new : rows;
    }
    const int extent = lrows > 0 ? (lrows - 1) * (int)row_bytes + NH * RB : 0;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(kbase + (int64_t)blk * block_bytes), (short)0, extent, kBufferWord3);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(vbase + (int64_t)blk * block_bytes), (short)0, extent, kBufferWord3);
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      st.k[i] = BufVec<16>::template load<kNt>(rk, roff[i]);
      st.v[i] = BufVec<16>::template load<kNt>(rv, roff[i]);
    }
    if constexpr (Q8) {
      const int sext = rows > 0 ? NSC * 2 : 0;
      const int64_t sblk = (int64_t)blk * sgroups * 32 + shead;
      const __amdgpu_buffer_rsrc_t skr = __builtin_amdgcn_make_buffer_rsrc(
          (void *)(reinterpret_cast<const char *>(kscale) + sblk), (short)0, sext, kBufferWord3);
      const __amdgpu_buffer_rsrc_t svr = __builtin_amdgcn_make_buffer_rsrc(
          (void *)(reinterpret_cast<const char *>(vscale) + sblk), (short)0, sext, kBufferWord3);
      if constexpr (NSC <= 64) {
        st.ks = __builtin_amdgcn_raw_buffer_load_b16(skr, (uint32_t)(sidx * 2), 0, 0);
        st.vs = __builtin_amdgcn_raw_buffer_load_b16(svr, (uint32_t)(sidx * 2), 0, 0);
        if ((sidx & 15) >= rows) st.ks = st.vs = 0;  // slots past the context may hold any scale
      } else {
        st.ks = __builtin_amdgcn_raw_buffer_load_b32(skr, (uint32_t)(sidx * 2), 0, 0);
        st.vs = __builtin_amdgcn_raw_buffer_load_b32(svr, (uint32_t)(sidx * 2), 0, 0);
        // entries sidx and sidx + 1 are slots (sidx & 15) and (sidx & 15) + 1 of one group
        const uint32_t keep = ((sidx & 15) >= rows ? 0u : 0xffffu) | ((sidx & 15) + 1 >= rows ? 0u : 0xffff0000u);
        st.ks &= keep;
        st.vs &= keep;
      }
    }
  };

  auto compute_tile = [&](int b, const Stage &st) __attribute__((always_inline)) {
    // Stage K (as loaded) and V (as f16) in LDS, row order, one region per head.
#pragma unroll
    for (int i = 0; i < NLD; ++i) {
      const int r = RPI * i + prow;
      *reinterpret_cast<u32x4 *>(sk[ph] + r * KPITCH + pc * 16) = st.k[i];
      if constexpr (Q8) {
        *reinterpret_cast<h8 *>(sv[ph] + r * VPITCH + pc * 32) = i8x8_to_h8(u32x2{st.v[i].x, st.v[i].y});
        *reinterpret_cast<h8 *>(sv[ph] + r * VPITCH + pc * 32 + 16) = i8x8_to_h8(u32x2{st.v[i].z, st.v[i].w});
      } else {
        *reinterpret_cast<u32x4 *>(sv[ph] + r * VPITCH + pc * 16) = st.v[i];
      }
    }
    if constexpr (!Q8) {
      // The fused new row (loaded as zeros: outside the tile's extent) is
      // overwritten from registers (every lane writes its piece; lanes of
      // different rows write the same bytes).
      if (b == cur.b_new) {
        *reinterpret_cast<u32x4 *>(sk[ph] + cur.r_new * KPITCH + pc * 16) = nk;
        *reinterpret_cast<u32x4 *>(sv[ph] + cur.r_new * VPITCH + pc * 16) = nv;
      }
    }
    if constexpr (Q8) {
      if constexpr (NSC <= 64) {
        ssc[0][sidx] = (uint16_t)st.ks;
        ssc[1][sidx] = (uint16_t)st.vs;
      } else {
        *reinterpret_cast<uint32_t *>(&ssc[0][sidx]) = st.ks;
        *reinterpret_cast<uint32_t *>(&ssc[1][sidx]) = st.vs;
      }
    }
    KV ka[NH][KS];
#pragma unroll
    for (int a = 0; a < NH; ++a)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        ka[a][ks] = *reinterpret_cast<const KV *>(sk[a] + lr * KPITCH + (32 * ks + 8 * lq) * (int)sizeof(T));

    // Scores of tokens 4 lq + i, column lr: every kv head's product lands in
    // the columns of its own query heads.
    f32x4 s;
    if constexpr (Q8) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        f32x4 c = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int a = 0; a < NH; ++a) c = __builtin_amdgcn_mfma_f32_16x16x32_f16(i8x8_to_h8_biased(ka[a][ks]), qb[a][ks], c, 0, 0, 0);
        const h4 d = *reinterpret_cast<const h4 *>(&ssc[0][(my_head * KS + ks) * 16 + 4 * lq]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float t = c[i] - qbias[ks];
          s[i] = ks == 0 ? (float)d[i] * t : __builtin_fmaf((float)d[i], t, s[i]);
        }
      }
    } else {
      s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int a = 0; a < NH; ++a)
          s = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, ka[a][ks]), qb[a][ks], s, 0, 0, 0);
    }
    float sc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) sc[i] = s[i] + dpp<0x140>(s[i]);  // hi + lo (row_mirror: lane ^ 15)
    if (qscaled) {  // uniform: heads beyond the f16 range entered the product as Q' 2^-e
#pragma unroll
      for (int i = 0; i < 4; ++i) sc[i] *= qmul;
    }
    const int valid = (int)(cur.tok1 - (int64_t)b * 16);  // rows of this tile inside the context
    if (valid < 16) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (4 * lq + i >= valid) sc[i] = -INFINITY;
    }

    // Softmax against the column's common reference, raised (with the
    // accumulators rescaled) only when a score exceeds it by the slack. The
    // maxima are NaN-propagating (v_maximum3_f32, no canonicalisation): a
    // NaN score makes the column's output NaN either way.
    const float lmax = __builtin_elementwise_maximum(__builtin_elementwise_maximum(sc[0], sc[1]),
                                                     __builtin_elementwise_maximum(sc[2], sc[3]));
    if (__builtin_amdgcn_ballot_w64(lmax > m_thr)) {
      float mx = __builtin_fmaxf(lmax, __shfl_xor(lmax, 16));
      mx = __builtin_fmaxf(mx, __shfl_xor(mx, 32));
      if (mx > m_thr) {
        const float alpha = __builtin_amdgcn_exp2f(m_ref - mx);
        m_ref = mx;
        m_thr = mx + kDecodeSlack;
        m_off = mx;
        l_run *= alpha;
#pragma unroll
        for (int a = 0; a < OS; ++a)
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) oacc[a][dt] *= alpha;
      }
    }
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f(sc[i] - m_off);
    l_run += (p[0] + p[1]) + (p[2] + p[3]);

    // O^T += V_a^T P'_a^T for each kv head a of the wave, per 16-row tile
    // of d; P'_a holds the weights of a's query heads (zero elsewhere) and,
    // for q8_0, the V scale of the tile's 32-element group.
    h4 pf = {};
    if constexpr (!Q8) pf = weight_parts(p, lo_mult);
#pragma unroll
    for (int g = 0; g < KS; ++g) {
      h4 pw = pf;
      if constexpr (Q8) {
        const h4 d = *reinterpret_cast<const h4 *>(&ssc[1][(my_head * KS + g) * 16 + 4 * lq]);
        pw = weight_parts_scaled(p, d, lo_m2);
      }
      h4 pb[NH];
#pragma unroll
      for (int a = 0; a < NH; ++a) pb[a] = (NH == 1 || OS > 1 || a == my_head) ? pw : h4{};
#pragma unroll
      for (int dt = 2 * g; dt < 2 * g + 2; ++dt)
#pragma unroll
        for (int a = 0; a < NH; ++a) {
          const hf4 v = lds_read_tr(sv[a] + (4 * lq + (lr >> 2)) * VPITCH + (dt * 16 + 4 * (lr & 3)) * 2);
          f32x4 &acc = oacc[OS > 1 ? a : 0][dt];
          acc = __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h4, v), pb[a], acc, 0, 0, 0);
        }
    }
  };

  // The lane's own head's column sums, in place (the accumulators are reset
  // or dead afterwards): oacc[0] holds the numerators of rows d = 16 dt +
  // 4 lq + i of query head lr (the hi lanes), l_run the column's sum.
  auto reduce_acc = [&]() __attribute__((always_inline)) {
    if constexpr (OS > 1) {
#pragma unroll
      for (int a = 1; a < OS; ++a)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) oacc[0][dt] = a == my_head ? oacc[a][dt] : oacc[0][dt];
    }
    // Column sums over the four lane rows; hi + lo parts of the numerators.
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) oacc[0][dt][i] += dpp<0x140>(oacc[0][dt][i]);
  };
  // Partial (numerators, reference, sum) of partition it.part, after reduce_acc.
  auto write_partial = [&](const Item &it) __attribute__((always_inline)) {
    if (!hi_lane) return;
    const int64_t qh = it.qi * n_heads + (int64_t)kvh0 * G + lr;
    const int64_t pi = qh * max_parts + it.part;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      *reinterpret_cast<f32x4 *>(part_o + pi * HD + 16 * dt + 4 * lq) = oacc[0][dt];
    if (lq == 0) {
      part_ml[2 * pi] = m_ref;
      part_ml[2 * pi + 1] = l_run;
    }
  };

  // The item's result: the output (one partition) or the partial of its last
  // partition.
  auto finish = [&](const Item &it) __attribute__((always_inline)) {
    reduce_acc();
    if (!hi_lane) return;  // lane (j, lq) holds rows d = 16 dt + 4 lq + i of the wave's query head j
    if (it.np > 1) {
      write_partial(it);
      return;
    }
    auto &o = oacc[0];
    const int64_t qh = it.qi * n_heads + (int64_t)kvh0 * G + lr;
    // one partition: this wave writes the output
    const int npre = pre_parts ? pre_parts[it.qi] : 0;
    if (npre > 0) {
      // Fold the query's group partials (numerator, reference, sum) into
      // the wave's own, four partials per round (indices clamped to the
      // last partial, with weight 0 past it): one round of loads brings
      // their references, sums and numerators together, and the running
      // reference is raised to the round's maximum as it goes (the
      // accumulators rescaled), so no separate pass finds the maximum.
      const float *pml = pre_ml + qh * max_pre_parts * 2;
      float mref = m_ref;
      for (int p0 = 0; p0 < npre; p0 += 4) {
        f32x4 po[4][DT];
        float pm[4], pl[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int pc = p0 + u < npre ? p0 + u : npre - 1;
          const float *src = pre_o + (qh * max_pre_parts + pc) * HD + 4 * lq;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) po[u][dt] = *reinterpret_cast<const f32x4 *>(src + 16 * dt);
          pm[u] = pml[2 * pc];
          pl[u] = pml[2 * pc + 1];
        }
        float mx = mref;
#pragma unroll
        for (int u = 0; u < 4; ++u) mx = __builtin_fmaxf(mx, pm[u]);  // clamped: a repeat, harmless
        // While every reference seen is -inf (empty partials, empty own
        // range) the running reference stays -inf and nothing is added; it
        // never takes a finite placeholder that later rounds would use as a
        // floor.
        const bool any = mx != -INFINITY;
        const float a0 = any ? __builtin_amdgcn_exp2f(mref - mx) : 1.f;
        l_run *= a0;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[dt] *= a0;
        mref = any ? mx : mref;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float a = p0 + u < npre && any ? __builtin_amdgcn_exp2f(pm[u] - mref) : 0.f;
          l_run += pl[u] * a;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) o[dt] += po[u][dt] * a;
        }
      }
    }
    const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      *reinterpret_cast<f32x4 *>(out + qh * HD + 16 * dt + 4 * lq) =
          l_run > 0.f ? o[dt] * inv : f32x4{0.f, 0.f, 0.f, 0.f};
  };

  // STAGES - 1 tiles in flight while one is computed; loads past the last
  // tile read nothing (extent 0).
  f32x4 qr[2 * KS], kr[2], vr[2];
  make_item(cur, qr, kr, vr);
  if (!cur.valid) return;
  LTKV_STAMP(1);
  reset();
  int b = cur.b0;
  // Table entries are read one tile ahead of their loads (the first ones
  // together), so no load waits on its own scalar read.
  auto entry_of = [&](int bb) __attribute__((always_inline)) { return bb < cur.b1 ? scalar_read(cur.tab, bb) : 0; };
  auto load_b = [&](int bb, int32_t entry, Stage &st) __attribute__((always_inline)) {
    load_tile(entry, cur.qi, cur.tok1, cur.b_new, cur.r_new, bb < cur.b1, bb, st);
  };
  // More tiles left, more priority: the waves of a SIMD end their items
  // together instead of one after the other (Qwen2.5-7B step 197.5-198.0
  // -> 189.7-191.6 us; thresholds 40 / 16 or 32 / 12 tiles measured within
  // 1% of these; one wave per SIMD, as at the Llama-3-8B shape, is unchanged).
  auto wave_priority = [&](int left) __attribute__((always_inline)) {
    if (left > 48) __builtin_amdgcn_s_setprio(2);
    else if (left > 24) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
  };
  // The tile loop stops at `stop`: the item's end or, inside a run, the end
  // of the current partition. There the partition's partial goes to the
  // wave's LDS slot cur.part - cur.p0 (fewer than kRunSlots: runs are at
  // most kRunSlots + 1 partitions) and the next partition starts from empty
  // accumulators (the tiles in flight are the next partition's). One test
  // per tile, as for the item's end alone: a separate test per tile cost the
  // Qwen2.5-7B step 3% (the tiles' work no longer overlapped across it).
  auto part_stop = [&]() __attribute__((always_inline)) {
    const int e = (cur.part + 1) * cur.pt_tiles;
    return e < cur.b1 ? e : cur.b1;
  };
  int stop = part_stop();
  auto next_part = [&]() __attribute__((always_inline)) {
    if constexpr (RUNS) {
      reduce_acc();
      const int slot = cur.part - cur.p0;
      if (hi_lane) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) srun_o[wv][slot][dt][lq * NQ + lr] = oacc[0][dt];
        if (lq == 0) {
          srun_ml[wv][slot][lr][0] = m_ref;
          srun_ml[wv][slot][lr][1] = l_run;
        }
      }
      reset();
      ++cur.part;
      stop = part_stop();
    }
  };
  // After tile b - 1 (b incremented): false when the item is done.
  auto more = [&]() __attribute__((always_inline)) {
    if constexpr (RUNS) {
      if (b >= stop) {
        if (b >= cur.b1) return false;
        next_part();
      }
      return true;
    } else {
      return b < cur.b1;
    }
  };
  if (b < cur.b1) {
    if constexpr (STAGES == 3) {
      Stage s0, s1, s2;
      const int32_t e0 = entry_of(b), e1 = entry_of(b + 1);
      int32_t en = entry_of(b + 2);
      load_b(b, e0, s0);
      load_b(b + 1, e1, s1);
      LTKV_STAMP(2);
      convert_q(qr, qb, qbias);
      commit_new(cur, kr, vr, nk, nv);
      for (;;) {
        wave_priority(cur.b1 - b);
        int32_t ea = entry_of(b + 3);
        load_b(b + 2, en, s2);
        compute_tile(b, s0);
        LTKV_STAMP_ONCE(3);
        ++b;
        if (!more()) break;
        en = entry_of(b + 3);
        load_b(b + 2, ea, s0);
        compute_tile(b, s1);
        ++b;
        if (!more()) break;
        ea = entry_of(b + 3);
        load_b(b + 2, en, s1);
        compute_tile(b, s2);
        ++b;
        if (!more()) break;
        en = ea;
      }
    } else {
      Stage s0, s1;
      const int32_t e0 = entry_of(b);
      int32_t en = entry_of(b + 1);
      load_b(b, e0, s0);
      LTKV_STAMP(2);
      convert_q(qr, qb, qbias);
      commit_new(cur, kr, vr, nk, nv);
      for (;;) {
        wave_priority(cur.b1 - b);
        int32_t ea = entry_of(b + 2);
        load_b(b + 1, en, s1);
        compute_tile(b, s0);
        LTKV_STAMP_ONCE(3);
        ++b;
        if (!more()) break;
        en = entry_of(b + 2);
        load_b(b + 1, ea, s0);
        compute_tile(b, s1);
        ++b;
        if (!more()) break;
      }
    }
  }
  LTKV_STAMP(4);
  finish(cur);
  // The run's staged partials (partitions p0 .. part - 1).
  if (RUNS && hi_lane) {
    const int64_t qh = cur.qi * n_heads + (int64_t)kvh0 * G + lr;
    for (int slot = 0; slot < cur.part - cur.p0; ++slot) {  // uniform
      const int64_t pi = qh * max_parts + cur.p0 + slot;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        *reinterpret_cast<f32x4 *>(part_o + pi * HD + 16 * dt + 4 * lq) = srun_o[wv][slot][dt][lq * NQ + lr];
      if (lq == 0) {
        part_ml[2 * pi] = srun_ml[wv][slot][lr][0];
        part_ml[2 * pi + 1] = srun_ml[wv][slot][lr][1];
      }
    }
  }
#ifdef LTKV_TIMELINE
  LTKV_STAMP(5);
  tl_[6] = (unsigned long long)(cur.b1 - cur.b0);
  tl_[7] = (unsigned long long)cur.qi << 16 | (unsigned long long)cur.part << 8 | (unsigned long long)kvh0;
  if (lane == 0 && gw < kTimelineWaves)
    for (int i = 0; i < 8; ++i) g_timeline[gw * 8 + i] = tl_[i];
#endif
  if (fault_q >= 0) report_fault(status, kFaultTable, fault_q);
}

// Plain decode attention of up to kOrderMaxQueries queries takes its items
// longest first; planned launches (query maps, group partials) keep query
// order.
inline bool decode_ordered(const AttnArgs &a) {
  return !a.qmap && !a.pre_parts && a.n > 1 && a.n <= kOrderMaxQueries;
}

// One wave per item (a partition of NH kv heads of one query), kDecodeWaves
// consecutive items per work-group; the grid is rounded up to whole
// work-groups and the waves past the last item leave at once.
template <typename T, int HD, int G, int NH, bool RUNS>
hipError_t launch_attn_mfma_k(const PoolGeom &g, const AttnArgs &a, int slots, int pair_items, hipStream_t s) {
  constexpr int nw = kDecodeWaves;
  const unsigned grid = (unsigned)((a.n * (a.n_kv_heads / NH) * a.max_parts + nw - 1) / nw);
  attn_mfma_kernel<T, HD, G, NH, RUNS><<<grid, 64 * nw, 0, s>>>(
      static_cast<const T *>(a.k_layer), static_cast<const T *>(a.v_layer), a.q, a.tables, a.table_stride,
      a.lens, a.out, a.part_o, a.part_ml, a.n_kv_heads, g.n_blocks, g.block_stride, g.slot_stride,
      g.head_stride, a.scale * kLog2e, a.part_tokens, a.split, a.max_parts, a.pre_parts, a.qmap,
      static_cast<const uint16_t *>(a.k_scale), static_cast<const uint16_t *>(a.v_scale), a.rows, a.n_rows,
      a.max_len, a.pre_o, a.pre_ml, a.max_pre_parts, a.new_slots, a.new_k, a.new_v, a.new_stride,
      static_cast<T *>(const_cast<void *>(a.k_layer)), static_cast<T *>(const_cast<void *>(a.v_layer)), a.n,
      decode_ordered(a) ? 1 : 0, slots, pair_items, a.status);
  return launch_merge<HD>(a, s, true);
}

// Ordered launches of f16 two-head waves whose grid holds at least twice the
// waves the chip holds at once take the kernel with runs of partitions (the
// lengths then decide the run length; it may still be 1); the others the
// kernel without. Both give the same bits.
template <typename T, int HD, int G, int NH>
hipError_t launch_attn_mfma_t(const PoolGeom &g, const AttnArgs &a, hipStream_t s) {
  constexpr int nw = kDecodeWaves;
  if constexpr (NH == 2 && !std::is_same_v<T, int8_t>) {
    // Waves the chip holds at once (work-groups per CU from the kernel's
    // registers and LDS).
    static const int per_cu = [] {
      int blocks = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, attn_mfma_kernel<T, HD, G, NH, true>, 64 * nw,
                                                       0) != hipSuccess)
        blocks = 0;
      return blocks * nw;
    }();
    const int64_t slots = (int64_t)per_cu * a.cu_count;
    if (decode_ordered(a) && slots > 0 && a.n * (a.n_kv_heads / NH) * a.max_parts >= 2 * slots)
      return launch_attn_mfma_k<T, HD, G, NH, true>(g, a, (int)slots, 0, s);
  }
  // Work-groups per CU of the kernel without runs; with two, the items of
  // the work-groups the chip starts with are paired longest with shortest.
  static const int wg_per_cu = [] {
    int blocks = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, attn_mfma_kernel<T, HD, G, NH, false>, 64 * nw, 0) !=
        hipSuccess)
      blocks = 0;
    return blocks;
  }();
  const int pair_items = wg_per_cu == 2 ? 2 * a.cu_count * nw / (a.n_kv_heads / NH) : 0;
  return launch_attn_mfma_k<T, HD, G, NH, false>(g, a, 0, pair_items, s);
}

template <typename T, int HD, int G>
hipError_t launch_attn16_t(const PoolGeom &g, const AttnArgs &a, hipStream_t s) {
  const unsigned grid = (unsigned)(a.n * a.n_kv_heads * a.max_parts);
  attn16_kernel<T, HD, G, kAttnWaves><<<grid, 64 * kAttnWaves, 0, s>>>(
      static_cast<const T *>(a.k_layer), static_cast<const T *>(a.v_layer), a.q, a.tables,
      a.table_stride, a.lens, a.out, a.part_o, a.part_ml, a.n_kv_heads, g.n_blocks,
      g.block_stride, g.slot_stride, g.head_stride, a.scale * kLog2e, a.part_tokens, a.max_parts,
      a.pre_parts, a.qmap, a.rows, a.n_rows, a.max_len, a.status);
  return launch_merge<HD>(a, s, false);
}

template <typename T, int HD, int G>
hipError_t launch_attn_t(const PoolGeom &g, const AttnArgs &a, hipStream_t s) {
  const unsigned grid = (unsigned)(a.n * a.n_kv_heads * a.max_parts);
  attn_kernel<T, HD, G><<<grid, 256, 0, s>>>(
      static_cast<const T *>(a.k_layer), static_cast<const T *>(a.v_layer), a.q, a.tables,
      a.table_stride, a.lens, a.out, a.part_o, a.part_ml, a.n_kv_heads, g.n_blocks,
      g.block_stride, g.slot_stride, g.head_stride, a.scale * kLog2e, a.part_tokens, a.max_parts,
      a.pre_parts, a.qmap, a.rows, a.n_rows, a.max_len, a.status);
  return launch_merge<HD>(a, s, false);
}

// f16 and q8_0 pools take the matrix-core kernel. f32 pools (no f32 MFMA
// form keeps the products exact at this rate) stay on the VALU: 16 lanes per
// row (f32 x 64, f16 x 128) take attn16_kernel, other rows attn_kernel. f16
// pools take the VALU kernels too when the caller asks for them
// (LTKV_ENGINE_VALU: the bandwidth-bound design without matrix cores, kept
// to measure the two against each other).
template <typename T, int HD>
constexpr bool kRow16 = HD / Tile<T>::E == 16;

template <typename T, int HD, int G>
hipError_t launch_attn_g(const PoolGeom &g, const AttnArgs &a, hipStream_t s) {
  if constexpr (std::is_same_v<T, _Float16>) {
    if (a.valu) {
      if constexpr (kRow16<T, HD>) return launch_attn16_t<T, HD, G>(g, a, s);
      else return launch_attn_t<T, HD, G>(g, a, s);
    }
  }
  if constexpr (!std::is_same_v<T, float>) {
    if constexpr (G <= 4) {
      if (a.n_kv_heads % 2 == 0) return launch_attn_mfma_t<T, HD, G, 2>(g, a, s);
    }
    return launch_attn_mfma_t<T, HD, G, 1>(g, a, s);
  }
  else if constexpr (kRow16<T, HD>)
    return launch_attn16_t<T, HD, G>(g, a, s);
  else
    return launch_attn_t<T, HD, G>(g, a, s);
}

template <typename T, int HD>
hipError_t launch_attn_hd(const PoolGeom &g, const AttnArgs &a, hipStream_t s) {
  switch (a.n_heads / a.n_kv_heads) {
    case 1: return launch_attn_g<T, HD, 1>(g, a, s);
    case 2: return launch_attn_g<T, HD, 2>(g, a, s);
    case 3: return launch_attn_g<T, HD, 3>(g, a, s);
    case 4: return launch_attn_g<T, HD, 4>(g, a, s);
    case 5: return launch_attn_g<T, HD, 5>(g, a, s);
    case 6: return launch_attn_g<T, HD, 6>(g, a, s);
    case 7: return launch_attn_g<T, HD, 7>(g, a, s);
    case 8: return launch_attn_g<T, HD, 8>(g, a, s);
    default: return hipErrorInvalidValue;
  }
}


// ----------------------------------------------------------------------------
// Shared-prefix (cascade) attention. The members of a prefix-sharing group
// read the same leading blocks, so their query rows (every member x every
// query head of a kv head) attend to those blocks once, together: with
// hundreds of rows per K/V row the work is GEMM-shaped, and it runs on MFMA
// (v_mfma_f32_16x16x32_f16) instead of once per member on the VALU:
//   S^T[token][row] = K Q^T   A = K rows (LDS), B = Q^T (registers)
//   O^T[d][row]    += V^T P^T A = V^T (LDS transpose reads), B = P^T, whose
//                             layout is the C layout of S^T
// Q and P are f32; each is split into f16 hi + lo parts (hi + lo equals the
// f32 value to about 2^-22 relative) and both products accumulate in f32,
// so scores and sums keep f32 accuracy over the exact f16 K and V. The
// result of a work-group is a partial (numerator, max, sum) per row for its
// token range, folded into each member's output by attn_merge_kernel.
//
// Work-group: 4 waves x 32 rows (two 16-row tiles per wave); K and V are
// staged 32 tokens at a time through double-buffered LDS. MFMA and VALU
// instructions of the waves of a SIMD do not overlap on this chip, so the
// kernel keeps the VALU count per score low rather than interleaving.
// Operand layouts of v_mfma_f32_16x16x32_f16 (lane l, j = 0..7, i = 0..3):
// A[l % 16][8 (l / 16) + j], B[8 (l / 16) + j][l % 16], D[4 (l / 16) + i][l % 16].
// ds_read_b64_tr_b16 within each 16-lane group: lane i, element j is element
// i % 4 of the 8 bytes addressed by lane 4 j + i / 4.
// ----------------------------------------------------------------------------

constexpr int kMqChunk = 32;       // tokens per staging step
constexpr int kMqTabMax = kMqMaxRange / 16;  // table entries of one job's token range
constexpr float kMqSlack = 8.f;    // log2 headroom of the softmax reference

// x = hi + lo with hi = f16(x) and lo = f16(x - hi); x - hi is exact in f32.
// m1 holds -1 in a register the compiler cannot see through, so x - hi stays
// one v_fma_mix_f32 on the packed f16 hi (a literal -1 turns it into a
// conversion back to f32 and a subtraction), and hi is converted once, two
// elements per v_cvt_pk_f16_f32.
__device__ __forceinline__ void split_hl(const float (&x)[8], h8 &hi, h8 &lo, float m1) {
#pragma unroll
  for (int j = 0; j < 8; j += 2) {
    const h2 h = __builtin_convertvector(f32x2{x[j], x[j + 1]}, h2);
    hi[j] = h[0];
    hi[j + 1] = h[1];
    lo[j] = (_Float16)__builtin_fmaf((float)h[0], m1, x[j]);
    lo[j + 1] = (_Float16)__builtin_fmaf((float)h[1], m1, x[j + 1]);
  }
}

// -1.f in a register that the optimiser treats as unknown (for split_hl).
__device__ __forceinline__ float opaque_minus_one() {
  float m1 = -1.f;
  asm volatile("" : "+v"(m1));
  return m1;
}


// Work-group: eight waves of 32 query rows (256 rows), two waves per SIMD;
// each staged K/V chunk serves all 256 rows.
constexpr int kMqWaves = 8;
constexpr int kMqStages = 3;  // LDS stages (and register sets) of the chunk ring

// F16P: the products take Q and the softmax weights P rounded to f16, one
// MFMA each (no lo parts): half the MFMA work and no split of P on the VALU,
// at ~2^-12 relative error per operand (opt-in, LTKV_PLAN_F16_PRODUCTS).
template <typename T, int HD, bool F16P>
__global__ void __launch_bounds__(64 * kMqWaves, 2)
mq_attn_kernel(const T *__restrict__ kpool, const T *__restrict__ vpool,
               const float *__restrict__ q, const int32_t *__restrict__ tables,
               const MqJob *__restrict__ jobs, int n_jobs, const int32_t *__restrict__ members,
               float *__restrict__ pre_o, float *__restrict__ pre_ml, float *__restrict__ out,
               int n_heads, int group,
               int64_t n_blocks, int64_t block_stride, int64_t slot_stride, float qscale,
               int max_pre_parts, const uint16_t *__restrict__ kscale,
               const uint16_t *__restrict__ vscale) {
  constexpr bool Q8 = std::is_same_v<T, int8_t>;
  constexpr int KS = HD / 32;                // k steps of the score product (q8_0: scale groups)
  constexpr int DT = HD / 16;                // 16-wide d tiles of the output
  // LDS bytes per staged row, f16. The pads keep the score product's K
  // reads (16 bytes a lane) and the transposing V reads (8 bytes a lane,
  // four rows x four columns per 16 lanes) free of bank conflicts: at
  // head_dim 128, 0 SQ_LDS_BANK_CONFLICT cycles with these pitches, 12.4 M
  // per prefill 8 x 512 dispatch with K rows padded by 16 bytes (prefill
  // 1-2% slower), 25 M with V rows padded by 16 or 48, 87-99 M with either
  // unpadded. head_dim 64 keeps its K pad of 16 bytes.
  constexpr int ROWK = HD * 2 + (HD == 128 ? 32 : 16);
  constexpr int ROWV = HD * 2 + 32;
  constexpr int VPR = HD * (int)sizeof(T) / 16;  // 16-byte vectors per pool row
  constexpr int NT = 64 * kMqWaves;  // threads
  constexpr int NV = kMqChunk * VPR;         // vectors per chunk, K and V each
  constexpr int NPT = (NV + NT - 1) / NT;    // vectors per thread per chunk, K and V each
  static_assert(NV % NT == 0 || NV < NT, "chunk must split over the threads");
  static_assert(64 / VPR <= 16, "a wave's rows of a chunk must lie in one block");
  constexpr int NSC = KS * kMqChunk;         // q8_0 scale entries of a chunk, K or V
  static_assert(!Q8 || 2 * NSC <= NT, "one scale entry per thread");
  __shared__ __attribute__((aligned(16))) char smk[kMqStages][kMqChunk * ROWK];  // [stage] K rows as f16
  __shared__ __attribute__((aligned(16))) char smv[kMqStages][kMqChunk * ROWV];  // [stage] V rows as f16
  // q8_0: [stage][K, V][group][token] scales of the staged chunk
  __shared__ __attribute__((aligned(16))) uint16_t ssm[kMqStages][2][Q8 ? NSC : 1];
  // The job's blocks: {byte offset lo, hi, load extent, block id}; extent 0
  // for blocks outside the pool. kMqTabPad entries past the range read as
  // {0, 0, 0, -1} (no load, no block), enough for the ring's loads past the
  // last chunk.
  constexpr int kMqTabPad = 10;
  __shared__ __attribute__((aligned(16))) i32x4 stab[kMqTabMax + kMqTabPad];

  // The job list is ordered by work-group id (XCD placement is the host's);
  // empty jobs pad it.
  if ((int)blockIdx.x >= n_jobs) return;
  const MqJob jb = jobs[blockIdx.x];
  if (jb.n_members <= 0) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lr = lane & 15, lq = lane >> 4;
  const int rows = jb.n_members * group;
  const bool active = wave * 32 < rows;  // wave-uniform

  // This lane's query row in each of the wave's two row tiles, as the B
  // operand Q^T: 8 consecutive d of k step ks at d = 32 ks + 8 lq.
  h8 qh[2][KS], ql[2][KS];
  int limit[2];
  int64_t slot[2], qrow[2];
  float qmul[2];  // per row tile: the lane's row's factor 2^e for its scores (q_range_exp)
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int r = wave * 32 + rt * 16 + lr;
    float x[KS][8];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) x[ks][e] = 0.f;
    limit[rt] = 0;
    slot[rt] = -1;
    qrow[rt] = 0;
    if (r < rows) {
      const int m = r / group, hh = r - m * group;
      const int qi = members[2 * (jb.member0 + m)];
      limit[rt] = members[2 * (jb.member0 + m) + 1];
      const int64_t qh_idx = (int64_t)qi * n_heads + (int64_t)jb.kvh * group + hh;
      qrow[rt] = qh_idx;
      slot[rt] = qh_idx * max_pre_parts + jb.part;
      const float *qp = q + qh_idx * HD + 8 * lq;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const f32x4 a = *reinterpret_cast<const f32x4 *>(qp + 32 * ks);
        const f32x4 b = *reinterpret_cast<const f32x4 *>(qp + 32 * ks + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          x[ks][e] = a[e] * qscale;
          x[ks][4 + e] = b[e] * qscale;
        }
      }
    }
    // a row beyond the f16 range enters the products as x 2^-e (q_range_exp);
    // its 128 (64) elements lie in lanes lr + 16 lq
    float amax = 0.f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) amax = __builtin_fmaxf(amax, __builtin_fabsf(x[ks][e]));
    amax = __builtin_fmaxf(amax, __shfl_xor(amax, 16));
    amax = __builtin_fmaxf(amax, __shfl_xor(amax, 32));
    const int qex = q_range_exp(amax);
    const float qinv = __builtin_ldexpf(1.f, -qex);
    qmul[rt] = __builtin_ldexpf(1.f, qex);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) x[ks][e] *= qinv;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if constexpr (F16P) {
#pragma unroll
        for (int e = 0; e < 8; ++e) qh[rt][ks][e] = (_Float16)x[ks][e];
      } else {
        split_hl(x[ks], qh[rt][ks], ql[rt][ks], -1.f);
      }
    }
  }
  // Whether any row of the wave entered the products scaled (uniform): its
  // score accumulators then start at 0 and take s 2^e - reference afterwards.
  const bool qscaled = __builtin_amdgcn_ballot_w64(qmul[0] != 1.f || qmul[1] != 1.f) != 0;
  // q8_0 K is staged as 1152 + k (exact in f16): 1152 times the row's sum of
  // each k step of Q (hi + lo) comes off every score of that step.
  float qbias[2][KS];
  if constexpr (Q8) {
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        float t = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) t += (float)qh[rt][ks][e] + (F16P ? 0.f : (float)ql[rt][ks][e]);
        t += __shfl_xor(t, 16);
        t += __shfl_xor(t, 32);
        qbias[rt][ks] = 1152.f * t;
      }
  }

  // Staging: token tok's row of this kv head is one contiguous HD-element
  // run; tokens at or past t1 stage as zeros. q8_0 rows are converted to f16
  // on the way into LDS (K biased as above, V exact), with their scales.
  // The job's block-table entries are read once into LDS with each block's
  // byte offset and load extent, so a chunk's buffer descriptors cost an LDS
  // read and a 64-bit add, with no scalar-memory wait.
  const int32_t *tab = tables + jb.table;
  const int tb0 = jb.t0 >> 4;                       // first table entry of the range
  int ntab = (jb.t1 - jb.t0 + 15) >> 4;             // entries of the range
  ntab = ntab < kMqTabMax ? ntab : kMqTabMax;        // (the planner keeps ranges within it)
  const uint32_t row_bytes = (uint32_t)(slot_stride * (int64_t)sizeof(T));
  for (int i = threadIdx.x; i < ntab + kMqTabPad; i += NT) {
    i32x4 e = i32x4{0, 0, 0, -1};
    if (i < ntab) {
      const int32_t blk = tab[tb0 + i];
      const int valid = jb.t1 - (tb0 + i) * 16;  // rows of the block inside the range (> 0)
      const bool ok = blk >= 0 && blk < n_blocks;
      const int64_t off = ok ? (int64_t)blk * block_stride * (int64_t)sizeof(T) : 0;
      const int ext = ok ? ((valid < 16 ? valid : 16) - 1) * (int)row_bytes + HD * (int)sizeof(T) : 0;
      e = i32x4{(int32_t)(uint32_t)off, (int32_t)(off >> 32), ext, ok ? blk : -1};
    }
    stab[i] = e;
  }
  const int64_t head_off = (int64_t)jb.kvh * HD;
  // Chunks start on block boundaries (t0 % 32 == 0) and a wave's share of a
  // chunk lies in one block. K/V rows go through buffer descriptors whose
  // extent ends at t1: rows past it (and chunks past the range) load as
  // zeros with no branch and no traffic.
  const int64_t sgroups = slot_stride >> 5;         // q8_0 scale groups per pool row
  const int64_t shead = (int64_t)jb.kvh * (HD / 32);  // first scale group of this kv head
  // Table entry e (wave-uniform) as a byte offset and a load extent.
  auto block_desc = [&](int e, int64_t &off, int &ext) {
    e = e < kMqTabMax + kMqTabPad ? e : kMqTabMax + kMqTabPad - 1;
    const i32x4 v = stab[e];
    off = (int64_t)(((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane(v.y) << 32) |
                    (uint32_t)__builtin_amdgcn_readfirstlane(v.x));
    ext = __builtin_amdgcn_readfirstlane(v.z);
  };
  // Chunk j of K (KIND 0) or V (KIND 1) into registers: a wave's rows of the
  // chunk lie in one of its two blocks, entry 2 j or 2 j + 1.
  auto load_part = [&](auto kind, int j, u32x4 (&r)[NPT], uint32_t &sc) {
    constexpr int KIND = decltype(kind)::value;
    const char *pool = reinterpret_cast<const char *>((KIND == 0 ? kpool : vpool) + head_off);
    const int c0 = jb.t0 + j * kMqChunk;
    if constexpr (Q8) {
      // thread t < NSC: entry t (group t / 32, token t % 32) of the chunk's scales
      sc = 0;
      if ((int)threadIdx.x < NSC) {
        const int e = (int)threadIdx.x, tok = c0 + e % kMqChunk;
        const int te = 2 * j + ((tok >> 4) & 1);
        const int32_t blk = stab[te < kMqTabMax + kMqTabPad ? te : kMqTabMax + kMqTabPad - 1].w;
        if (blk >= 0 && tok < jb.t1) {
          const uint16_t *sp = KIND == 0 ? kscale : vscale;
          sc = sp[((int64_t)blk * sgroups + shead + e / kMqChunk) * 16 + (tok & 15)];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < NPT; ++u) {
      const int idx = threadIdx.x + NT * u;
      if (NV < NT && idx >= NV) break;  // wave-uniform: NV is a multiple of 64
      const int row = idx / VPR, col = idx - row * VPR;
      int64_t off;
      int ext;
      block_desc(2 * j + ((__builtin_amdgcn_readfirstlane(row) >> 4) & 1), off, ext);
      const __amdgpu_buffer_rsrc_t rs =
          __builtin_amdgcn_make_buffer_rsrc((void *)(pool + off), (short)0, ext, kBufferWord3);
      const uint32_t voff = (uint32_t)((c0 + row) & 15) * row_bytes + (uint32_t)col * 16;
      r[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, 0, 0));
    }
  };
  auto store_part = [&](auto kind, int st, const u32x4 (&r)[NPT], uint32_t sc) {
    constexpr int KIND = decltype(kind)::value;
#pragma unroll
    for (int u = 0; u < NPT; ++u) {
      const int idx = threadIdx.x + NT * u;
      if (NV < NT && idx >= NV) break;
      const int row = idx / VPR, col = idx - row * VPR;
      char *base = KIND == 0 ? smk[st] + row * ROWK : smv[st] + row * ROWV;
      if constexpr (Q8) {
        char *d = base + col * 32;
        if constexpr (KIND == 0) {
          *reinterpret_cast<h8 *>(d) = i8x8_to_h8_biased(u32x2{r[u].x, r[u].y});
          *reinterpret_cast<h8 *>(d + 16) = i8x8_to_h8_biased(u32x2{r[u].z, r[u].w});
        } else {
          *reinterpret_cast<h8 *>(d) = i8x8_to_h8(u32x2{r[u].x, r[u].y});
          *reinterpret_cast<h8 *>(d + 16) = i8x8_to_h8(u32x2{r[u].z, r[u].w});
        }
      } else {
        *reinterpret_cast<u32x4 *>(base + col * 16) = r[u];
      }
    }
    if constexpr (Q8) {
      if ((int)threadIdx.x < NSC) ssm[st][KIND][threadIdx.x] = (uint16_t)sc;
    }
  };
  using KPart = std::integral_constant<int, 0>;
  using VPart = std::integral_constant<int, 1>;

  // Chunks wholly inside every valid row's visible range need no masking
  // (rows past n_members are never stored and need none).
  int lim_min = jb.t1;
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
    if (slot[rt] >= 0) lim_min = limit[rt] < lim_min ? limit[rt] : lim_min;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int other = __shfl_xor(lim_min, off);
    lim_min = other < lim_min ? other : lim_min;
  }
  lim_min = __builtin_amdgcn_readfirstlane(lim_min);  // the same in every lane now

  // Softmax reference per row: p = 2^(s - m_ref) with s <= m_ref + kMqSlack,
  // so p <= 2^kMqSlack (exact in the f16 hi/lo split). The reference is
  // raised (and the accumulators rescaled) only when a score exceeds it by
  // more than the slack, which after the first chunk is rare; the fast path
  // needs no cross-lane exchange. The score product starts its accumulators
  // at -m_ref (0 while the row has no reference), so they hold s - m_ref.
  float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};
  // f16 products of f16 pools take the row sums on the matrix cores: one
  // more value tile of ones (lsum, every element the row's sum of the same
  // f16 weights the numerator takes; prefill 8 x 512 235 -> 231 us). The
  // other forms add them on the vector ALU (l_run, spread over the row's
  // four lanes): f32-accurate products would need two more products per
  // row tile beside their doubled ones (359 -> 369 us), and q8_0 pools
  // scale the weights per V group.
  constexpr bool LM = F16P && !Q8;
  f32x4 lsum[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  f32x4 o[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt][0] = o[dt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto mref = [&](int rt) { return m_run[rt] == -INFINITY ? 0.f : m_run[rt]; };
  // Start of the score accumulators, -reference, changed only where the
  // reference is raised.
  f32x4 sinit[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  // A chunk's row maximum (less the reference) above this takes the raise
  // path: the slack with a reference, -inf without one (any score sets it).
  float thr[2] = {-INFINITY, -INFINITY};
  const float m1 = opaque_minus_one();

  // Scores of 32 tokens (two 16-token tiles) x this wave's 32 rows, from the
  // K rows of LDS stage st, less the rows' references. Consecutive MFMAs go
  // to different accumulators.
  // K fragments of LDS stage st: the A operands of the score product.
  auto read_k = [&](int st, h8 (&a)[KS][2]) {
    const char *ks_base = smk[st];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
        a[ks][tt] = *reinterpret_cast<const h8 *>(ks_base + (tt * 16 + lr) * ROWK + (32 * ks + 8 * lq) * 2);
  };
  auto score = [&](int st, const h8 (&ka)[KS][2], f32x4 (&sc)[2][2]) {
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) sc[0][rt] = sc[1][rt] = qscaled ? f32x4{0.f, 0.f, 0.f, 0.f} : sinit[rt];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const h8 a[2] = {ka[ks][0], ka[ks][1]};
      if constexpr (Q8) {
        // each k step is one scale group: its product is scaled by the
        // token's K scale d after the bias comes off, d (sum - bias)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const h4 d = *reinterpret_cast<const h4 *>(&ssm[st][0][ks * kMqChunk + tt * 16 + 4 * lq]);
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) {
            f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[tt], qh[rt][ks], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            if constexpr (!F16P) c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[tt], ql[rt][ks], c, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 4; ++i) sc[tt][rt][i] = __builtin_fmaf((float)d[i], c[i] - qbias[rt][ks], sc[tt][rt][i]);
          }
        }
      } else {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int rt = 0; rt < 2; ++rt)
            sc[tt][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[tt], qh[rt][ks], sc[tt][rt], 0, 0, 0);
        if constexpr (!F16P) {
#pragma unroll
          for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
              sc[tt][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[tt], ql[rt][ks], sc[tt][rt], 0, 0, 0);
        }
      }
    }
    if (qscaled) {  // uniform: rows beyond the f16 range entered as Q 2^-e
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
#pragma unroll
          for (int i = 0; i < 4; ++i) sc[tt][rt][i] = __builtin_fmaf(sc[tt][rt][i], qmul[rt], sinit[rt][i]);
    }
  };

  // Online softmax of one chunk's scores into the P^T operand. This lane
  // holds tokens 4 lq + i and 16 + 4 lq + i of its row; k slot j of P^T is
  // token j < 4 ? 4 lq + j : 16 + 4 lq + j - 4. f16 products of f16 pools
  // take P rounded to f16 (ph, summed by the products); otherwise P stays
  // f32 (pf) for the split or the q8_0 scales, and its row sums are added
  // here.
  constexpr bool PH = F16P && !Q8;
  auto softmax = [&](f32x4 (&sc)[2][2], int c0, float (&pf)[2][8], h8 (&ph)[2]) {
    float lmax[2];
    if (c0 + kMqChunk > lim_min) {  // uniform: the chunk crosses a row's limit
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const int lim = (jb.t1 < limit[rt] ? jb.t1 : limit[rt]) - c0;  // visible tokens of the chunk
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (tt * 16 + 4 * lq + i >= lim) sc[tt][rt][i] = -INFINITY;
      }
    }
    // NaN-propagating maxima (v_maximum3_f32, no operand canonicalisation):
    // a NaN score makes its row's output NaN either way.
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      lmax[rt] = sc[0][rt][0];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) lmax[rt] = __builtin_elementwise_maximum(lmax[rt], sc[tt][rt][i]);
    }
    const bool over = (lmax[0] > thr[0]) | (lmax[1] > thr[1]);
    if (__builtin_amdgcn_ballot_w64(over)) {
      // Raise the reference of the rows some lane found above it; the row
      // max is exchanged over the row's four lanes, so the decision and the
      // new reference are the same in all of them.
#pragma unroll
      for (int rt = 0; rt < 2; ++rt) {
        const float m0 = mref(rt);
        float mx = lmax[rt] + m0;
        mx = __builtin_fmaxf(mx, __shfl_xor(mx, 16));
        mx = __builtin_fmaxf(mx, __shfl_xor(mx, 32));
        const bool raise = mx > m_run[rt] + kMqSlack;
        const float alpha = raise ? __builtin_amdgcn_exp2f(m_run[rt] - mx) : 1.f;
        const float shift = raise ? m0 - mx : 0.f;
        m_run[rt] = raise ? mx : m_run[rt];
        const float nm = -mref(rt);
        sinit[rt] = f32x4{nm, nm, nm, nm};
        thr[rt] = m_run[rt] == -INFINITY ? -INFINITY : kMqSlack;
        l_run[rt] *= alpha;
        lsum[rt] *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[dt][rt] *= alpha;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) sc[tt][rt] += shift;
      }
    }
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) pf[rt][tt * 4 + i] = __builtin_amdgcn_exp2f(sc[tt][rt][i]);
      if constexpr (PH) {
#pragma unroll
        for (int j = 0; j < 8; ++j) ph[rt][j] = (_Float16)pf[rt][j];
      } else if constexpr (!LM) {
        float ps = pf[rt][0];
#pragma unroll
        for (int j = 1; j < 8; ++j) ps += pf[rt][j];
        l_run[rt] += ps;
      }
    }
  };

  // O^T += V^T P^T over the V rows of LDS stage st.
  auto pv = [&](int st, const float (&pf)[2][8], const h8 (&php)[2]) {
    const char *vs_base = smv[st];
    h8 ph[2], pl[2];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      if constexpr (Q8) {
        if (dt % 2 == 0) {  // a new scale group: P' = P times the token's V scale
          const int g = dt / 2;
          const h4 d0 = *reinterpret_cast<const h4 *>(&ssm[st][1][g * kMqChunk + 4 * lq]);
          const h4 d1 = *reinterpret_cast<const h4 *>(&ssm[st][1][g * kMqChunk + 16 + 4 * lq]);
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) {
            float x[8];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              x[j] = pf[rt][j] * (float)d0[j];
              x[4 + j] = pf[rt][4 + j] * (float)d1[j];
            }
            if constexpr (F16P) {
#pragma unroll
              for (int j = 0; j < 8; ++j) ph[rt][j] = (_Float16)x[j];
            } else {
              split_hl(x, ph[rt], pl[rt], m1);
            }
          }
        }
      } else if (dt == 0) {
#pragma unroll
        for (int rt = 0; rt < 2; ++rt) {
          if constexpr (F16P) {
            ph[rt] = php[rt];
          } else {
            split_hl(pf[rt], ph[rt], pl[rt], m1);
          }
        }
      }
      // V^T operand: d = 16 dt + lr, tokens 4 lq + j (j < 4) and 16 + 4 lq + j - 4.
      const int col = (dt * 16 + 4 * (lr & 3)) * 2;
      const u32x2 a0 = __builtin_bit_cast(u32x2, lds_read_tr(vs_base + (4 * lq + (lr >> 2)) * ROWV + col));
      const u32x2 a1 = __builtin_bit_cast(u32x2, lds_read_tr(vs_base + (16 + 4 * lq + (lr >> 2)) * ROWV + col));
      const h8 a = __builtin_bit_cast(h8, u32x4{a0.x, a0.y, a1.x, a1.y});
#pragma unroll
      for (int rt = 0; rt < 2; ++rt)
        o[dt][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ph[rt], o[dt][rt], 0, 0, 0);
      if constexpr (!F16P) {
#pragma unroll
        for (int rt = 0; rt < 2; ++rt)
          o[dt][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, pl[rt], o[dt][rt], 0, 0, 0);
      }
      if constexpr (LM) {
        if (dt == 0) {  // the row sums: V^T rows of ones
          const h8 ones = h8{1.f16, 1.f16, 1.f16, 1.f16, 1.f16, 1.f16, 1.f16, 1.f16};
#pragma unroll
          for (int rt = 0; rt < 2; ++rt) {
            lsum[rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, ph[rt], lsum[rt], 0, 0, 0);
            if constexpr (!F16P) lsum[rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pl[rt], lsum[rt], 0, 0, 0);
          }
        }
      }
    }
  };

  // Chunk loop over a ring of three LDS stages and three register sets: in
  // iteration c the wave computes chunk c (stage c % 3), stores chunk c + 2
  // (loaded two iterations earlier) into stage (c + 2) % 3, whose chunk c - 1
  // every wave finished before the last barrier, and loads chunk c + 4. The
  // stores are issued early and the loads have two iterations to land, so
  // the barrier that ends the iteration waits on neither (prefill 8 x 512:
  // 406 -> 392 us against two stages; q8_0 pools ~3% slower). Measured and
  // dropped: reading chunk c + 1's K fragments during chunk c's value product
  // (f16 products 3% slower); staging K one chunk ahead of V so that the next
  // chunk's score product overlaps this chunk's softmax (5-10% slower);
  // skewing each wave by half a chunk (chunk c + 1's scores beside chunk c's
  // weight split, chunk c's values beside chunk c + 1's exponentials, the
  // issue order pinned with sched_group_barrier: prefill 8 x 512 375 -> 392
  // us, 249 -> 285 us with f16 products).
  // Chunks past the range load as zeros (empty extent), so every step is
  // unconditional.
  const int nch = (jb.t1 - jb.t0 + kMqChunk - 1) / kMqChunk;
  struct Staged {
    u32x4 k[NPT], v[NPT];
    uint32_t sk, sv;
  };
  auto load_pair = [&](int j, Staged &r) {  // K(j) and V(j)
    load_part(KPart{}, j, r.k, r.sk);
    load_part(VPart{}, j, r.v, r.sv);
  };
  auto store_pair = [&](int st, const Staged &r) {
    store_part(KPart{}, st, r.k, r.sk);
    store_part(VPart{}, st, r.v, r.sv);
  };
  Staged r0, r1, r2;
  __syncthreads();  // the table entries
  load_pair(0, r0);
  load_pair(1, r1);
  load_pair(2, r2);
  store_pair(0, r0);
  store_pair(1, r1);
  load_pair(3, r0);
  __syncthreads();
  // ST: stage of chunk c (c % 3); ld: the set for chunk c + 4; sto: chunk c + 2's.
  auto iter = [&](auto stc, int c, Staged &ld, Staged &sto) {
    constexpr int ST = decltype(stc)::value;
    load_pair(c + 4, ld);
    store_pair((ST + 2) % kMqStages, sto);
    if (active) {
      f32x4 sc[2][2];
      float pf[2][8];
      h8 ph[2], ka[KS][2];
      read_k(ST, ka);
      score(ST, ka, sc);
      softmax(sc, jb.t0 + c * kMqChunk, pf, ph);
      pv(ST, pf, ph);
    }
    __syncthreads();
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  for (int c = 0; c < nch; c += 3) {
    iter(S0{}, c, r1, r2);
    if (c + 1 < nch) iter(S1{}, c + 1, r2, r0);
    if (c + 2 < nch) iter(S2{}, c + 2, r0, r1);
  }

  // Partial per row: the row's sum (lsum, or l_run spread over its four
  // lanes).
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    float l;
    if constexpr (LM) {
      l = lsum[rt][0];
    } else {
      l = l_run[rt];
      l += __shfl_xor(l, 16);
      l += __shfl_xor(l, 32);
    }
    if (slot[rt] >= 0 && jb.direct) {  // the row's only contribution: normalised output
      const float inv = l > 0.f ? 1.f / l : 0.f;
      float *po = out + qrow[rt] * HD + 4 * lq;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<f32x4 *>(po + dt * 16) = o[dt][rt] * inv;
    } else if (slot[rt] >= 0) {
      float *po = pre_o + slot[rt] * HD + 4 * lq;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) *reinterpret_cast<f32x4 *>(po + dt * 16) = o[dt][rt];
      if (lq == 0) {
        pre_ml[2 * slot[rt]] = m_run[rt];
        pre_ml[2 * slot[rt] + 1] = l;
      }
    }
  }
}

// ----------------------------------------------------------------------------
// Generic forms for the shapes the kernels above do not cover. The reference
// takes any shape (model.rs:401-402 reads head_dim and the group from the
// model; its own cache test uses kv_dim 4, kv.rs:202-229): rows whose byte
// length is not a multiple of 16 move element by element, and attention with
// a head_dim other than 64 / 128 or a group above 8 runs on the vector ALU
// with one work-group per (query, query head). They are correct for any
// shape and serve the families the tuned kernels do not; the tuned kernels
// stay the path for every shape they cover.
// ----------------------------------------------------------------------------

// Append of one element of K and of V per thread (any kv_dim).
template <int ELEM>
__global__ void __launch_bounds__(256)
write_any_kernel(uint8_t *__restrict__ kpool, uint8_t *__restrict__ vpool, const int32_t *__restrict__ slots,
                 const float *__restrict__ k, const float *__restrict__ v, int64_t n, int64_t src_stride,
                 int64_t kv_dim, int64_t n_slots, const int32_t *__restrict__ order, int64_t n_rows) {
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t i = gid / kv_dim;
  if (i >= n) return;
  const int64_t e = gid - i * kv_dim;
  const int64_t row = order ? order[i] : i;  // write_kernel's order
  if (order && (row < 0 || row >= n_rows)) return;
  const int32_t s = slots[row];
  if (s < 0 || (int64_t)s >= n_slots) return;
  const int64_t dst = (int64_t)s * kv_dim + e;
  const float kx = k[row * src_stride + e], vx = v[row * src_stride + e];
  if constexpr (ELEM == 2) {
    reinterpret_cast<uint16_t *>(kpool)[dst] = (uint16_t)f16_bits(kx);
    reinterpret_cast<uint16_t *>(vpool)[dst] = (uint16_t)f16_bits(vx);
  } else {
    reinterpret_cast<float *>(kpool)[dst] = kx;
    reinterpret_cast<float *>(vpool)[dst] = vx;
  }
}

// Gather with element-wise moves: work-group = (sequence, table entry, K or V).
template <typename E>
__global__ void __launch_bounds__(256)
gather_any_kernel(const E *__restrict__ kpool, const E *__restrict__ vpool, const int32_t *__restrict__ tables,
                  int64_t table_stride, const int32_t *__restrict__ lens, const int64_t *__restrict__ out_offsets,
                  E *__restrict__ kout, E *__restrict__ vout, int64_t n_blocks, int64_t kv_dim,
                  int32_t *__restrict__ status) {
  const int is_v = (int)(blockIdx.x & 1);
  const int64_t entry = blockIdx.x >> 1;
  const int64_t seq = entry / table_stride;
  const int64_t j = entry - seq * table_stride;
  int64_t len = lens[seq];
  if (len > table_stride * 16) len = table_stride * 16;
  const int64_t start = j * 16;
  if (start >= len) return;
  const int64_t rows = len - start < 16 ? len - start : 16;
  const int32_t blk = tables[seq * table_stride + j];
  if (blk < 0 || blk >= n_blocks) {  // kv.rs:147 panics here; nothing is copied
    if (threadIdx.x == 0 && status) {
      __hip_atomic_fetch_or(status, kFaultTable, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      status[1] = (int32_t)seq;
    }
    return;
  }
  const E *src = (is_v ? vpool : kpool) + (int64_t)blk * 16 * kv_dim;
  E *dst = (is_v ? vout : kout) + (out_offsets[seq] + start) * kv_dim;
  for (int64_t i = threadIdx.x; i < rows * kv_dim; i += 256) dst[i] = src[i];
}

constexpr int kAnyThreads = 256;
constexpr int kAnyMaxHeadDim = 1024;  // four output elements per thread
constexpr int kAnyD = kAnyMaxHeadDim / kAnyThreads;

// Block-wide max / sum over the 256 threads (every thread gets it).
template <bool MAX>
__device__ __forceinline__ float block_reduce(float x, float *red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float y = __shfl_xor(x, off, 64);
    x = MAX ? __builtin_fmaxf(x, y) : x + y;
  }
  __syncthreads();  // red may still be read by the previous reduction
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  const float a = red[0], b = red[1], c = red[2], d = red[3];
  return MAX ? __builtin_fmaxf(__builtin_fmaxf(a, b), __builtin_fmaxf(c, d)) : (a + b) + (c + d);
}

// Element e of a pool row of cell `cell` (block * 16 + slot) as f32: f16 and
// f32 as stored, q8_0 as d * q (quant byte q + 128, scale d of the element's
// 32-element group, [block][kv_dim / 32][16 slots]).
template <typename T>
__device__ __forceinline__ float pool_elem(const T *pool, const uint16_t *scales, int64_t cell, int64_t kv_dim,
                                           int64_t e) {
  if constexpr (std::is_same_v<T, int8_t>) {
    const int q = (int)(uint8_t)pool[cell * kv_dim + e] - 128;
    const uint16_t d = scales[((cell >> 4) * (kv_dim >> 5) + (e >> 5)) * 16 + (cell & 15)];
    return (float)q * (float)__builtin_bit_cast(_Float16, d);
  } else {
    return (float)pool[cell * kv_dim + e];
  }
}

// Work-group = (query, query head): 256 tokens per round, one score per
// thread (a dot product over head_dim), softmax of the round against the
// running reference (exp2 domain), then each thread accumulates up to four
// output elements d = t + 256 k over the round's tokens.
template <typename T>
__global__ void __launch_bounds__(kAnyThreads)
attn_any_kernel(const T *__restrict__ kpool, const T *__restrict__ vpool, const uint16_t *__restrict__ kscale,
                const uint16_t *__restrict__ vscale, const float *__restrict__ q, const int32_t *__restrict__ tables,
                int64_t table_stride, const int32_t *__restrict__ lens, float *__restrict__ out, int n_heads,
                int group, int head_dim, int64_t n_blocks, int64_t kv_dim, float qscale,
                const int32_t *__restrict__ rows, int64_t n_rows, int64_t max_len, const int32_t *__restrict__ qmap,
                int32_t *__restrict__ status) {
  __shared__ float sq[kAnyMaxHeadDim];
  __shared__ float sp[kAnyThreads];
  __shared__ int32_t sblk[kAnyThreads / 16];
  __shared__ float red[4];
  const int t = (int)threadIdx.x;
  const int h = (int)(blockIdx.x % n_heads);
  const int64_t qx = blockIdx.x / n_heads;
  const int64_t qi = qmap ? qmap[qx] : qx;
  const int64_t head_off = (int64_t)(h / group) * head_dim;
  int64_t len = lens[qi];
  if (len < 0) len = 0;
  if (len > max_len) len = max_len;
  const int64_t qh = qi * n_heads + h;
  for (int d = t; d < head_dim; d += kAnyThreads) sq[d] = q[qh * head_dim + d] * qscale;
  const int32_t *tab = table_of(tables, table_stride, rows, n_rows, qi);
  if (t < 64) check_table(tab, 0, (int)((len + 15) >> 4), n_blocks, rows, n_rows, qi, status);
  float m = -INFINITY, l = 0.f, o[kAnyD];
#pragma unroll
  for (int k = 0; k < kAnyD; ++k) o[k] = 0.f;
  for (int64_t t0 = 0; t0 < len; t0 += kAnyThreads) {
    const int n_tok = len - t0 < kAnyThreads ? (int)(len - t0) : kAnyThreads;
    if (t < (n_tok + 15) / 16) {
      int32_t blk = tab[(t0 >> 4) + t];
      if (blk < 0 || blk >= n_blocks) blk = 0;  // reported by check_table
      sblk[t] = blk;
    }
    __syncthreads();
    float sc = -INFINITY;
    if (t < n_tok) {
      const int64_t cell = (int64_t)sblk[t >> 4] * 16 + ((t0 + t) & 15);
      float acc = 0.f;
      for (int d = 0; d < head_dim; ++d) acc += sq[d] * pool_elem(kpool, kscale, cell, kv_dim, head_off + d);
      sc = acc;
    }
    const float mx = block_reduce<true>(sc, red);
    const float mn = __builtin_fmaxf(m, mx);  // finite: the round has a token
    const float alpha = __builtin_amdgcn_exp2f(m - mn);
    const float p = t < n_tok ? __builtin_amdgcn_exp2f(sc - mn) : 0.f;
    sp[t] = p;
    l = l * alpha + block_reduce<false>(p, red);
    m = mn;
#pragma unroll
    for (int k = 0; k < kAnyD; ++k) o[k] *= alpha;
    __syncthreads();
    for (int j = 0; j < n_tok; ++j) {
      const int64_t cell = (int64_t)sblk[j >> 4] * 16 + ((t0 + j) & 15);
      const float pj = sp[j];
#pragma unroll
      for (int k = 0; k < kAnyD; ++k) {
        const int d = t + kAnyThreads * k;
        if (d < head_dim) o[k] += pj * pool_elem(vpool, vscale, cell, kv_dim, head_off + d);
      }
    }
    __syncthreads();  // sblk and sp are rewritten next round
  }
  const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
  for (int k = 0; k < kAnyD; ++k) {
    const int d = t + kAnyThreads * k;
    if (d < head_dim) out[qh * head_dim + d] = o[k] * inv;
  }
}

// ----------------------------------------------------------------------------
// Resident block tables (step descriptor): in-place updates and the slot
// mapping of a batch's tokens.

// Update i is (row, col, value): tables[row][col] = value, or, with col ==
// -1, counts[row] = value (the row's table length in blocks). Entries outside
// the arrays are skipped.
__global__ void __launch_bounds__(256)
table_update_kernel(int32_t *__restrict__ tables, int32_t *__restrict__ counts, int64_t width,
                    int64_t n_rows, const int32_t *__restrict__ upd, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int32_t r = upd[3 * i], c = upd[3 * i + 1], v = upd[3 * i + 2];
  if (r < 0 || r >= n_rows) return;
  if (c == -1)
    counts[r] = v;
  else if (c >= 0 && c < width)
    tables[(int64_t)r * width + c] = v;
}

// The same for a step's few updates passed by value in the kernel arguments
// (no staging copy, no event).
__global__ void __launch_bounds__(256)
table_update_args_kernel(int32_t *__restrict__ tables, int32_t *__restrict__ counts, int64_t width,
                         int64_t n_rows, TableUpdates u) {
  const int i = (int)threadIdx.x;
  for (int k = i; k < u.n; k += 256) {
    const int32_t r = u.t[3 * k], c = u.t[3 * k + 1], v = u.t[3 * k + 2];
    if (r < 0 || r >= n_rows) continue;
    if (c == -1)
      counts[r] = v;
    else if (c >= 0 && c < width)
      tables[(int64_t)r * width + c] = v;
  }
}

// Takes the fault word: atomic exchanges with zero, so a fault raised by work
// running beside this kernel is either taken here or left for the next take.
__global__ void __launch_bounds__(64) status_take_kernel(int32_t *status) {
  if (threadIdx.x != 0) return;
  const int32_t bits = __hip_atomic_exchange(status, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const int32_t who = __hip_atomic_exchange(status + 1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  status[2] = bits;
  status[3] = who;
}

// Token i at position pos[i] of the sequence in row rows[i]: cell
// block * 16 + pos % 16 with block = tables[row][pos / 16] (kv.rs:95-121's
// (block, slot), flattened as the write kernels take it), or -1 when the row
// is outside the tables or pos / 16 is past the row's table length.
__global__ void __launch_bounds__(256)
slot_mapping_kernel(const int32_t *__restrict__ tables, const int32_t *__restrict__ counts,
                    int64_t width, int64_t n_rows, const int32_t *__restrict__ rows,
                    const int64_t *__restrict__ pos, int64_t n, int32_t *__restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int32_t r = rows[i];
  const int64_t p = pos[i];
  int32_t cell = -1;
  if (r >= 0 && r < n_rows && p >= 0) {
    const int64_t b = p >> 4;
    if (b < counts[r] && b < width) cell = tables[(int64_t)r * width + b] * 16 + (int32_t)(p & 15);
  }
  out[i] = cell;
}

}  // namespace

hipError_t launch_write_q8(const PoolGeom &g, void *k_layer, void *v_layer, void *k_scale,
                           void *v_scale, const int32_t *slots, const float *k, const float *v,
                           int64_t n, int64_t src_stride, hipStream_t s, const int32_t *order,
                           int64_t n_rows) {
  if (n <= 0) return hipSuccess;
  const int64_t threads = n * (g.kv_dim >> 2);
  const int64_t blocks = (threads + 255) / 256;
  write_q8_kernel<<<(unsigned)blocks, 256, 0, s>>>(
      static_cast<int8_t *>(k_layer), static_cast<int8_t *>(v_layer), static_cast<uint16_t *>(k_scale),
      static_cast<uint16_t *>(v_scale), slots, k, v, n, src_stride, g.kv_dim, g.n_blocks * 16, order, n_rows);
  return hipGetLastError();
}

template <int ELEM, bool STREAM>
hipError_t launch_write_form(const PoolGeom &g, void *k_layer, void *v_layer, const int32_t *slots,
                             const float *k, const float *v, int64_t n, int64_t src_stride, hipStream_t s,
                             const int32_t *order, int64_t n_rows) {
  constexpr int rows = STREAM ? 2 : 1;
  const int64_t threads = (n + rows - 1) / rows * (g.kv_dim >> 3);
  const int64_t blocks = (threads + 255) / 256;
  if (blocks >= (int64_t{1} << 32)) return hipErrorInvalidValue;
  uint8_t *kp = static_cast<uint8_t *>(k_layer), *vp = static_cast<uint8_t *>(v_layer);
  if constexpr (STREAM) {  // K, then V
    write_kernel<ELEM, true, 1><<<(unsigned)blocks, 256, 0, s>>>(kp, vp, slots, k, v, n, src_stride, g.kv_dim,
                                                                  g.n_blocks * 16, order, n_rows);
    write_kernel<ELEM, true, 2><<<(unsigned)blocks, 256, 0, s>>>(kp, vp, slots, k, v, n, src_stride, g.kv_dim,
                                                                  g.n_blocks * 16, order, n_rows);
  } else {
    write_kernel<ELEM, false><<<(unsigned)blocks, 256, 0, s>>>(kp, vp, slots, k, v, n, src_stride, g.kv_dim,
                                                                g.n_blocks * 16, order, n_rows);
  }
  return hipGetLastError();
}

hipError_t launch_write(const PoolGeom &g, void *k_layer, void *v_layer, const int32_t *slots,
                        const float *k, const float *v, int64_t n, int64_t src_stride,
                        hipStream_t s, const int32_t *order, int64_t n_rows) {
  if (n <= 0) return hipSuccess;
  if (g.kv_dim % 8 != 0) {  // rows of any length: element-wise
    const int64_t blocks = (n * g.kv_dim + 255) / 256;
    if (blocks >= (int64_t{1} << 32)) return hipErrorInvalidValue;
    if (g.elem == 2)
      write_any_kernel<2><<<(unsigned)blocks, 256, 0, s>>>(static_cast<uint8_t *>(k_layer),
                                                           static_cast<uint8_t *>(v_layer), slots, k, v, n,
                                                           src_stride, g.kv_dim, g.n_blocks * 16, order, n_rows);
    else
      write_any_kernel<4><<<(unsigned)blocks, 256, 0, s>>>(static_cast<uint8_t *>(k_layer),
                                                           static_cast<uint8_t *>(v_layer), slots, k, v, n,
                                                           src_stride, g.kv_dim, g.n_blocks * 16, order, n_rows);
    return hipGetLastError();
  }
  constexpr int64_t kLastLevelCache = 256ll << 20;  // MALL bytes
  const bool stream = n * (int64_t)g.kv_dim * 8 > kLastLevelCache;
  if (g.elem == 2)
    return stream ? launch_write_form<2, true>(g, k_layer, v_layer, slots, k, v, n, src_stride, s, order, n_rows)
                  : launch_write_form<2, false>(g, k_layer, v_layer, slots, k, v, n, src_stride, s, order, n_rows);
  return stream ? launch_write_form<4, true>(g, k_layer, v_layer, slots, k, v, n, src_stride, s, order, n_rows)
                : launch_write_form<4, false>(g, k_layer, v_layer, slots, k, v, n, src_stride, s, order, n_rows);
}

hipError_t launch_write_rope(const PoolGeom &g, void *k_layer, void *v_layer, const int32_t *slots,
                            const int32_t *positions, const float *k, const float *v, float *q,
                            int64_t n, int64_t src_stride, int64_t q_stride, int n_heads,
                            const RopeGeom &r, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  const int uph = r.head_dim >> 3;
  const int n_kv_heads = g.kv_dim / r.head_dim;
  const int64_t per = (int64_t)n_kv_heads * uph + (g.kv_dim >> 3) + (q ? (int64_t)n_heads * uph : 0);
  const int64_t blocks = (n * per + 255) / 256;
  if (g.elem == 2)
    write_rope_kernel<2><<<(unsigned)blocks, 256, 0, s>>>(
        static_cast<uint8_t *>(k_layer), static_cast<uint8_t *>(v_layer), slots, positions, k, v, q,
        n, src_stride, q_stride, g.kv_dim, n_kv_heads, n_heads, g.n_blocks * 16, r.table, r.max_pos,
        r.rope_dim, r.head_dim, r.neox);
  else
    write_rope_kernel<4><<<(unsigned)blocks, 256, 0, s>>>(
        static_cast<uint8_t *>(k_layer), static_cast<uint8_t *>(v_layer), slots, positions, k, v, q,
        n, src_stride, q_stride, g.kv_dim, n_kv_heads, n_heads, g.n_blocks * 16, r.table, r.max_pos,
        r.rope_dim, r.head_dim, r.neox);
  return hipGetLastError();
}

hipError_t launch_write_rope_q8(const PoolGeom &g, void *k_layer, void *v_layer, void *k_scale, void *v_scale,
                               const int32_t *slots, const int32_t *positions, const float *k, const float *v,
                               float *q, int64_t n, int64_t src_stride, int64_t q_stride, int n_heads,
                               const RopeGeom &r, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  const int64_t per = 2 * (int64_t)(g.kv_dim >> 3) + (q ? (int64_t)n_heads * (r.head_dim >> 3) : 0);
  const int64_t blocks = (n * per + 255) / 256;
  write_rope_q8_kernel<<<(unsigned)blocks, 256, 0, s>>>(
      static_cast<int8_t *>(k_layer), static_cast<int8_t *>(v_layer), static_cast<uint16_t *>(k_scale),
      static_cast<uint16_t *>(v_scale), slots, positions, k, v, q, n, src_stride, q_stride, g.kv_dim, n_heads,
      g.n_blocks * 16, r.table, r.max_pos, r.rope_dim, r.head_dim, r.neox);
  return hipGetLastError();
}

template <int THREADS, int VEC, bool LAYER_MAJOR>
hipError_t launch_copy_form(const PoolGeom &g, int n_layers, void *k_pool, void *v_pool, const int32_t *pairs,
                            int64_t n_pairs, hipStream_t s) {
  const int64_t block_bytes = g.block_stride * g.elem;
  const int64_t layer_bytes = g.n_blocks * block_bytes;
  constexpr int64_t chunk = (int64_t)THREADS * VEC * 16;
  const int chunks = (int)((block_bytes + chunk - 1) / chunk);
  const int64_t wgs = (int64_t)n_layers * n_pairs * 2 * chunks;
  if (wgs >= (int64_t{1} << 32)) return hipErrorInvalidValue;  // the grid's x dimension is 32 bits
  copy_blocks_kernel<THREADS, VEC, LAYER_MAJOR><<<(unsigned)wgs, THREADS, 0, s>>>(
      static_cast<uint8_t *>(k_pool), static_cast<uint8_t *>(v_pool), pairs, n_pairs, n_layers, g.n_blocks,
      block_bytes, layer_bytes, chunks);
  return hipGetLastError();
}

int64_t copy_max_pairs(const PoolGeom &g, int n_layers, bool bulk) {
  // one work-group per (pair, layer, K or V, chunk); the grid's x dimension is 32 bits
  const int64_t chunk = bulk ? (int64_t)kCopyBulkThreads * 16 : 256 * 2 * 16;
  const int64_t chunks = (g.block_stride * g.elem + chunk - 1) / chunk;
  return ((int64_t{1} << 32) - 1) / ((int64_t)n_layers * 2 * chunks);
}

hipError_t launch_copy_blocks(const PoolGeom &g, int n_layers, void *k_pool, void *v_pool,
                              const int32_t *pairs, int64_t n_pairs, bool bulk, hipStream_t s) {
  if (n_pairs <= 0) return hipSuccess;
  if (bulk) return launch_copy_form<kCopyBulkThreads, 1, true>(g, n_layers, k_pool, v_pool, pairs, n_pairs, s);
  return launch_copy_form<256, 2, false>(g, n_layers, k_pool, v_pool, pairs, n_pairs, s);
}

int64_t copy_order_buckets(int64_t n_blocks) { return (n_blocks >> kCopyOrderShift) + 1; }

hipError_t launch_copy_order(const int32_t *pairs, int64_t n_pairs, int64_t n_blocks, int32_t *counts,
                             int32_t *cursors, int32_t *sorted, hipStream_t s) {
  if (n_pairs <= 0) return hipSuccess;
  const unsigned grid = (unsigned)((n_pairs + 255) / 256);
  copy_order_count<<<grid, 256, 0, s>>>(pairs, n_pairs, n_blocks, counts);
  copy_order_scan<<<1, 1024, 0, s>>>(counts, cursors, (int)copy_order_buckets(n_blocks));
  copy_order_scatter<<<grid, 256, 0, s>>>(pairs, n_pairs, n_blocks, cursors, sorted);
  return hipGetLastError();
}

hipError_t launch_gather(const PoolGeom &g, const void *k_layer, const void *v_layer,
                         const int32_t *tables, int64_t table_stride, const int32_t *lens,
                         const int64_t *out_offsets, int64_t n, void *k_out, void *v_out,
                         int32_t *status, hipStream_t s) {
  if (n <= 0 || table_stride <= 0) return hipSuccess;
  const int64_t row_bytes = (int64_t)g.kv_dim * g.elem;
  if (row_bytes % 16 != 0) {  // rows of any length: element-wise
    const int64_t wgs = n * table_stride * 2;
    if (wgs >= (int64_t{1} << 32)) return hipErrorInvalidValue;
    if (g.elem == 2)
      gather_any_kernel<uint16_t><<<(unsigned)wgs, 256, 0, s>>>(
          static_cast<const uint16_t *>(k_layer), static_cast<const uint16_t *>(v_layer), tables, table_stride,
          lens, out_offsets, static_cast<uint16_t *>(k_out), static_cast<uint16_t *>(v_out), g.n_blocks,
          g.kv_dim, status);
    else
      gather_any_kernel<uint32_t><<<(unsigned)wgs, 256, 0, s>>>(
          static_cast<const uint32_t *>(k_layer), static_cast<const uint32_t *>(v_layer), tables, table_stride,
          lens, out_offsets, static_cast<uint32_t *>(k_out), static_cast<uint32_t *>(v_out), g.n_blocks,
          g.kv_dim, status);
    return hipGetLastError();
  }
  // A block's K (or V) is 16 rows = row_bytes 16-byte vectors.
  const int chunks = (int)((row_bytes + kGatherChunk - 1) / kGatherChunk);
  const int64_t wgs = n * table_stride * 2 * chunks;
  if (wgs * kGatherThreads >= (int64_t{1} << 32)) return hipErrorInvalidValue;
  gather_kernel<<<(unsigned)wgs, kGatherThreads, 0, s>>>(
      static_cast<const uint8_t *>(k_layer), static_cast<const uint8_t *>(v_layer), tables,
      table_stride, lens, out_offsets, static_cast<uint8_t *>(k_out),
      static_cast<uint8_t *>(v_out), g.n_blocks, row_bytes, chunks, status);
  return hipGetLastError();
}

hipError_t launch_table_update(int32_t *tables, int32_t *counts, int64_t width, int64_t n_rows,
                               const int32_t *upd, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  if ((n + 255) / 256 >= (int64_t{1} << 32)) return hipErrorInvalidValue;
  table_update_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(tables, counts, width, n_rows, upd, n);
  return hipGetLastError();
}

hipError_t launch_table_update_args(int32_t *tables, int32_t *counts, int64_t width, int64_t n_rows,
                                    const TableUpdates &u, hipStream_t s) {
  if (u.n <= 0) return hipSuccess;
  if (u.n > kTableUpdateArgs) return hipErrorInvalidValue;
  table_update_args_kernel<<<1, 256, 0, s>>>(tables, counts, width, n_rows, u);
  return hipGetLastError();
}

hipError_t launch_slot_mapping(const int32_t *tables, const int32_t *counts, int64_t width,
                               int64_t n_rows, const int32_t *rows, const int64_t *pos, int64_t n,
                               int32_t *out, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  if ((n + 255) / 256 >= (int64_t{1} << 32)) return hipErrorInvalidValue;
  slot_mapping_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(tables, counts, width, n_rows, rows,
                                                                  pos, n, out);
  return hipGetLastError();
}

hipError_t launch_status_take(int32_t *status, hipStream_t s) {
  status_take_kernel<<<1, 64, 0, s>>>(status);
  return hipGetLastError();
}

AttnWorkspace attention_workspace(int64_t n, int n_heads, int head_dim, int max_parts,
                                  bool always) {
  AttnWorkspace w{};
  if (max_parts <= 1 && !always) return w;
  const int64_t parts = n * n_heads * (int64_t)max_parts;
  w.part_o_off = 0;
  w.part_ml_off = parts * head_dim * 4;
  w.bytes = w.part_ml_off + parts * 2 * 4;
  return w;
}

bool attention_tuned(int elem, int head_dim, int group) {
  return (elem == 1 || elem == 2 || elem == 4) && (head_dim == 64 || head_dim == 128) && group >= 1 &&
         group <= 8;
}

bool attention_supported(int elem, int head_dim, int group) {
  return (elem == 1 || elem == 2 || elem == 4) && head_dim >= 1 && head_dim <= kAnyMaxHeadDim && group >= 1;
}

template <typename T>
hipError_t launch_attn_any_t(const PoolGeom &g, const AttnArgs &a, hipStream_t s) {
  const int64_t grid = a.n * a.n_heads;
  if (grid >= (int64_t{1} << 32)) return hipErrorInvalidValue;
  attn_any_kernel<T><<<(unsigned)grid, kAnyThreads, 0, s>>>(
      static_cast<const T *>(a.k_layer), static_cast<const T *>(a.v_layer),
      static_cast<const uint16_t *>(a.k_scale), static_cast<const uint16_t *>(a.v_scale), a.q, a.tables,
      a.table_stride, a.lens, a.out, a.n_heads, a.n_heads / a.n_kv_heads, a.head_dim, g.n_blocks, g.kv_dim,
      a.scale * kLog2e, a.rows, a.n_rows, a.max_len, a.qmap, a.status);
  return hipGetLastError();
}

hipError_t launch_decode_attention(const PoolGeom &g, const AttnArgs &a, hipStream_t s) {
  if (a.n <= 0) return hipSuccess;
  if (a.pass_empty && a.pre_parts) {  // only group partials to fold (a chunk cut into ranges)
    if (a.head_dim == 64) return launch_merge<64>(a, s, true);
    if (a.head_dim == 128) return launch_merge<128>(a, s, true);
    return hipErrorInvalidValue;
  }
  if (!attention_tuned(g.elem, a.head_dim, a.n_heads / a.n_kv_heads)) {
    // the generic kernel takes whole contexts: no partials, no group partials
    if (a.pre_parts || !attention_supported(g.elem, a.head_dim, a.n_heads / a.n_kv_heads))
      return hipErrorInvalidValue;
    if (g.elem == 1) return launch_attn_any_t<int8_t>(g, a, s);
    if (g.elem == 2) return launch_attn_any_t<_Float16>(g, a, s);
    return launch_attn_any_t<float>(g, a, s);
  }
  if (g.elem == 1) {
    if (a.head_dim == 64) return launch_attn_hd<int8_t, 64>(g, a, s);
    if (a.head_dim == 128) return launch_attn_hd<int8_t, 128>(g, a, s);
  } else if (g.elem == 2) {
    if (a.head_dim == 64) return launch_attn_hd<_Float16, 64>(g, a, s);
    if (a.head_dim == 128) return launch_attn_hd<_Float16, 128>(g, a, s);
  } else {
    if (a.head_dim == 64) return launch_attn_hd<float, 64>(g, a, s);
    if (a.head_dim == 128) return launch_attn_hd<float, 128>(g, a, s);
  }
  return hipErrorInvalidValue;
}

int attention_split(int elem, int group, int n_kv_heads) {
  if (!((elem == 1 || elem == 2) && group <= 4 && n_kv_heads % 2 == 0)) return 1;
  // Measured at the Llama-3-8B decode shape (64 queries): q8_0 waves of two
  // heads (256 B rows of K and of V) run fastest with each partition cut in
  // two; f16 waves of two heads (512 B rows, three tiles in flight) keep HBM
  // busy at one wave per SIMD and run fastest uncut. The cut depends on the
  // dtype and shape only, never on the batch, so a query's partitions (and
  // its result bits) stay those of its own length.
  return elem == 1 ? 2 : 1;
}

int attention_part_policy(int elem, int group, int n_kv_heads, bool valu) {
  // Measured at the Llama-3-8B decode shape (64 queries x U[2048, 4096], f16,
  // two kv heads a wave, four waves a work-group): 1024-token partitions for
  // queries over 2048 tokens (2-4 per query: about 900 waves, most of them
  // whole 64-tile partitions that end together, the last partition of a
  // query short) 127.9 us per fused step against 137.4-137.9 with four equal
  // partitions (1024 waves); 768- or 2048-token ones for every query 157 /
  // 178 us. The Qwen2.5-7B step (one kv head a wave) gains too (196.4-196.8
  // against 199.7 us). q8_0 pools (partitions cut in two) lose with it
  // (91.0 against 87.8 us), as does the vector-ALU engine (147.6 against
  // 144.8 us): they keep four equal partitions. A function of the shape and
  // engine only.
  (void)group;
  (void)n_kv_heads;
  return !valu && elem == 2 ? kPartCap : 0;
}

int mq_rows(int, int) { return 32 * kMqWaves; }

bool mq_supported(int elem, int head_dim, int group) {
  return (elem == 2 || elem == 1) && (head_dim == 64 || head_dim == 128) && group >= 1 &&
         group <= mq_rows(elem, head_dim);
}

hipError_t launch_mq_attention(const PoolGeom &g, const MqArgs &a, hipStream_t s) {
  if (a.n_jobs <= 0) return hipSuccess;
  const unsigned grid = (unsigned)a.n_jobs;
  const int group = a.n_heads / a.n_kv_heads;
  const float qscale = a.scale * kLog2e;
  const auto *ksc = static_cast<const uint16_t *>(a.k_scale);
  const auto *vsc = static_cast<const uint16_t *>(a.v_scale);
  auto run = [&](auto tag, auto hd) {
    using T = decltype(tag);
    constexpr int HD = decltype(hd)::value;
    auto go = [&](auto f16p) {
      mq_attn_kernel<T, HD, decltype(f16p)::value><<<grid, 64 * kMqWaves, 0, s>>>(
          static_cast<const T *>(a.k_layer), static_cast<const T *>(a.v_layer), a.q, a.tables, a.jobs,
          a.n_jobs, a.members, a.pre_o, a.pre_ml, a.out, a.n_heads, group, g.n_blocks, g.block_stride,
          g.slot_stride, qscale, a.max_pre_parts, ksc, vsc);
    };
    if (a.f16_products) go(std::true_type{});
    else go(std::false_type{});
    return hipGetLastError();
  };
  if (g.elem == 2 && a.head_dim == 128) return run(_Float16{}, std::integral_constant<int, 128>{});
  if (g.elem == 2 && a.head_dim == 64) return run(_Float16{}, std::integral_constant<int, 64>{});
  if (g.elem == 1 && a.head_dim == 128) return run(int8_t{}, std::integral_constant<int, 128>{});
  if (g.elem == 1 && a.head_dim == 64) return run(int8_t{}, std::integral_constant<int, 64>{});
  return hipErrorInvalidValue;
}

namespace {
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxScratchDevices] = {};
}  // namespace

hipError_t scratch_address(int device, void **ptr) {
  *ptr = nullptr;
  if (device < 0 || device >= kMaxScratchDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    if (cur != device) return hipErrorInvalidDevice;  // the lookup needs `device` current
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_scratch_ptr[device] = p;
  }
  *ptr = g_scratch_ptr[device];
  return hipSuccess;
}

}  // namespace ltkv

#ifdef LTKV_TIMELINE
// Copies the stamps of the last decode launch (n entries of the [wave][8]
// array) to host memory and clears them; profiling build only.
extern "C" __attribute__((visibility("default"))) int ltkv_timeline_read(unsigned long long *h, size_t n) {
  if (n > (size_t)kTimelineWaves * 8) n = (size_t)kTimelineWaves * 8;
  if (hipDeviceSynchronize() != hipSuccess) return -1;
  if (hipMemcpyFromSymbol(h, HIP_SYMBOL(g_timeline), n * 8, 0, hipMemcpyDeviceToHost) != hipSuccess) return -1;
  static unsigned long long zeros[4096];
  for (size_t i = 0; i < (size_t)kTimelineWaves * 8; i += 4096)
    if (hipMemcpyToSymbol(HIP_SYMBOL(g_timeline), zeros, sizeof zeros, i * 8, hipMemcpyHostToDevice) != hipSuccess)
      return -1;
  return 0;
}
#endif
