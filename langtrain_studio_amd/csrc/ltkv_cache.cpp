// Host side of the MI355X paged KV cache: block allocator, block tables,
// refcounted prefix sharing with copy-on-write, and the C ABI of ltkv.h.
//
// Metadata semantics follow engine/crates/native/src/kv.rs:15-187 exactly
// (same allocation order, same refcount rule for copy-on-write, same error
// messages), so block tables are identical to the reference's for the same
// call sequence. The K/V pools live in HBM; every device op is enqueued on
// the cache's stream, in call order.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/ltkv.h"
#include "ltkv_kernels.h"

static_assert(LTKV_NOALLOC_SCRATCH_BYTES == ltkv::kScratchBytes, "scratch size of ltkv.h and the kernels");

namespace {

// Caller copy batches from this many pairs on are bucketed by destination on
// the device before the copy (three extra launches, a few microseconds; at
// 131 072 pairs the copy runs ~13% faster in destination order).
constexpr size_t kCopyOrderMinPairs = 4096;

// Message of the last failing call on this thread: a fixed buffer, so that
// reporting an error never allocates.
thread_local char g_err[512];

int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char *what) {
  return fail(LTKV_ERR_HIP, "HIP error in %s: %s", what, hipGetErrorString(e));
}

int no_device() {
  return fail(LTKV_ERR_ARG, "metadata-only cache (LTKV_NO_DEVICE): device ops are unavailable");
}

#define HIP_TRY(call, what)              \
  do {                                   \
    hipError_t e_ = (call);              \
    if (e_ != hipSuccess) return hip_fail(e_, what); \
  } while (0)

struct Seq {
  std::vector<int32_t> blocks;  // kv.rs:30
  size_t len = 0;               // kv.rs:31
};

// Step descriptor of ltkv_plan_attention: host-built tables, uploaded once.
// Device arrays (int32, each 32-byte aligned inside one buffer): one table
// row per group [groups][gstride], the per-query pass's tables [n][sstride]
// and lengths [n], group partials per query [n], members [2 * n_members],
// jobs [n_jobs].
struct AttnPlan {
  bool valid = false;
  uint64_t gen = 0;
  size_t n = 0, n_heads = 0, head_dim = 0, stride = 0, sstride = 0;
  int max_pre_parts = 0, n_jobs = 0;
  int suffix_part = 0;  // partition tokens of the per-query pass when grouped
  uint64_t groups = 0, grouped = 0, shared_blocks = 0;
  bool groups_only = false;  // every query completed by its group: no per-query pass
  size_t n_pass = 0;         // queries of the per-query pass (the rest are completed by groups)
  size_t max_suffix = 0;     // longest remainder (tokens) of a per-query-pass query
  bool empty_with_groups = false;  // a query with group partials and no remainder
  bool pass_empty = false;         // every per-query-pass query is such a query
  bool f16_products = false;       // LTKV_PLAN_F16_PRODUCTS
  size_t off_tables = 0, off_stables = 0, off_slens = 0, off_pre = 0, off_qmap = 0,
         off_members = 0, off_jobs = 0, bytes = 0;
  std::vector<int32_t> host;  // the arrays above, in device layout
  uint8_t *d = nullptr, *h = nullptr;  // device buffer, pinned staging
  size_t cap = 0;
  hipEvent_t done = nullptr;
  bool in_flight = false;
};

// Switches to the cache's device for the scope of a call.
struct DeviceGuard {
  int prev = -1;
  bool ok = true;
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != dev) ok = hipSetDevice(dev) == hipSuccess;
  }
  ~DeviceGuard() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

}  // namespace

struct ltkv_cache {
  int device = 0;
  int dtype = LTKV_F16;
  size_t n_layers = 0, kv_dim = 0, n_blocks = 0, elem = 2;
  ltkv::PoolGeom geom{};
  void *k = nullptr, *v = nullptr;  // [layer][block][slot][kv_dim]
  // Q8_0: per-32-element f16 scales, [layer][block][slot][kv_dim / 32].
  void *ks = nullptr, *vs = nullptr;
  ltkv::PoolGeom sgeom{};  // the scale pools as a pool of 2-byte elements
  hipStream_t stream = nullptr;

  std::vector<uint32_t> refs;   // kv.rs:23
  std::vector<int32_t> free;    // kv.rs:24, back() pops first
  std::unordered_map<uint32_t, Seq> seqs;  // kv.rs:25
  uint64_t cow_copies = 0;

  // Copy-on-write pair staging: pinned host buffer -> device buffer.
  std::vector<int32_t> pending;  // (src, dst) pairs of the current claim
  std::vector<std::pair<int32_t, int32_t>> pending_sorted;  // (dst, src), flush scratch
  int32_t *h_pairs = nullptr, *d_pairs = nullptr;
  size_t pairs_cap = 0;  // pairs
  hipEvent_t pairs_done = nullptr;
  bool pairs_in_flight = false;
  // Destination ordering of large caller copy batches (ltkv_copy_blocks):
  // bucket counts (zero between calls), cursors and the reordered pairs.
  int32_t *d_order_counts = nullptr, *d_order_pairs = nullptr;
  size_t order_cap = 0;  // pairs

  // Fault word of the device ops (int32[4], zeroed at creation): kernels OR
  // fault bits (a block-table entry outside the pool, a fused append's cell
  // that is not the query's position len - 1) into word 0 and the query into
  // word 1; ltkv_synchronize takes them (words 2..3 receive what was taken).
  int32_t *d_status = nullptr;

  // Attention workspace (partition partials), grown on demand.
  uint8_t *ws = nullptr;
  size_t ws_bytes = 0;
  // The device's static scratch (ltkv_decode_attention_noalloc), looked up at
  // creation; shared by every cache on the device.
  uint8_t *scratch = nullptr;
  size_t attn_part_tokens = 0;  // 0 = automatic
  int attn_engine = LTKV_ENGINE_AUTO;

  // RoPE table (ltkv_rope_init): [max_pos][rope_dim / 2] of (cos, sin).
  float *rope = nullptr;
  ltkv::RopeGeom rope_geom{};

  // Bumped by every metadata change; a plan records the value it was built at.
  uint64_t gen = 0;
  AttnPlan plan;

  int device_count_cu = 256;

  // Resident block tables (the device step descriptor): one row per live
  // sequence, [rt_rows][rt_width] block ids plus [rt_rows] table lengths, kept
  // equal to `seqs` by uploading only the entries that changed (sync_tables).
  int32_t *d_rt = nullptr, *d_rt_nb = nullptr;
  size_t rt_rows = 0, rt_width = 0;             // device capacity
  std::unordered_map<uint32_t, int32_t> rt_row;  // live sequence -> row
  std::vector<uint32_t> rt_seq;                  // row -> sequence
  std::vector<char> rt_live;                     // row holds a live sequence
  std::vector<int32_t> rt_free;                  // released rows, reused last-in first-out
  std::vector<uint32_t> rt_lo, rt_hi;            // per row: changed entries [lo, hi)
  std::vector<char> rt_dirty;                    // per row: changed since the last sync
  std::vector<uint32_t> rt_nb;                   // per row: table length in blocks as last synced
  std::vector<int32_t> rt_dirty_rows;
  std::vector<int32_t> rt_upd;                   // (row, col, value) triples being built
  int32_t *h_rt_upd = nullptr, *d_rt_upd = nullptr;  // pinned staging -> device
  size_t rt_upd_cap = 0;                         // triples
  hipEvent_t rt_done = nullptr;
  bool rt_in_flight = false;
  uint64_t rt_uploaded = 0;                      // triples uploaded so far (statistics)

  size_t layer_elems() const { return n_blocks * LTKV_BLOCK * kv_dim; }
  uint8_t *k_layer(size_t l) const { return (uint8_t *)k + l * layer_elems() * elem; }
  uint8_t *v_layer(size_t l) const { return (uint8_t *)v + l * layer_elems() * elem; }
  bool q8() const { return dtype == LTKV_Q8_0; }
  size_t layer_scales() const { return n_blocks * LTKV_BLOCK * (kv_dim / 32); }
  uint16_t *k_scales(size_t l) const { return ks ? (uint16_t *)ks + l * layer_scales() : nullptr; }
  uint16_t *v_scales(size_t l) const { return vs ? (uint16_t *)vs + l * layer_scales() : nullptr; }

  bool alloc(int32_t *b) {  // kv.rs:67-74
    if (free.empty()) return false;
    *b = free.back();
    free.pop_back();
    refs[*b] = 1;
    return true;
  }
  void release(int32_t b) {  // kv.rs:76-81
    refs[b] -= 1;
    if (refs[b] == 0) free.push_back(b);
  }

  // Row of a live sequence in the resident tables, assigned on first use.
  int32_t rt_row_of(uint32_t seq) {
    auto it = rt_row.find(seq);
    if (it != rt_row.end()) return it->second;
    int32_t r;
    if (!rt_free.empty()) {
      r = rt_free.back();
      rt_free.pop_back();
    } else {
      r = (int32_t)rt_seq.size();
      rt_seq.push_back(0);
      rt_live.push_back(0);
      rt_lo.push_back(0);
      rt_hi.push_back(0);
      rt_dirty.push_back(0);
      rt_nb.push_back(0);
    }
    rt_row.emplace(seq, r);
    rt_seq[r] = seq;
    rt_live[r] = 1;
    return r;
  }
  void rt_touch(int32_t r, size_t lo, size_t hi) {  // entries [lo, hi) and the length changed
    if (!rt_dirty[r]) {
      rt_dirty[r] = 1;
      rt_dirty_rows.push_back(r);
      rt_lo[r] = (uint32_t)lo;
      rt_hi[r] = (uint32_t)hi;
    } else if (lo < hi) {
      if (rt_lo[r] >= rt_hi[r]) {
        rt_lo[r] = (uint32_t)lo;
        rt_hi[r] = (uint32_t)hi;
      } else {
        rt_lo[r] = std::min<uint32_t>(rt_lo[r], (uint32_t)lo);
        rt_hi[r] = std::max<uint32_t>(rt_hi[r], (uint32_t)hi);
      }
    }
  }
  void rt_mark(uint32_t seq, size_t lo, size_t hi) { rt_touch(rt_row_of(seq), lo, hi); }
  void rt_remove(uint32_t seq) {  // the sequence is gone: its row reads as empty
    auto it = rt_row.find(seq);
    if (it == rt_row.end()) return;
    const int32_t r = it->second;
    rt_row.erase(it);
    rt_live[r] = 0;
    rt_touch(r, 0, 0);
    rt_free.push_back(r);
  }

  // kv.rs:85-121 without the device copy: a copy-on-write is recorded in
  // `pending` and launched by the caller before any later device work.
  int append_meta(uint32_t seq, size_t pos, uint32_t *block, uint32_t *slot) {
    ++gen;
    Seq &s = seqs[seq];  // entry(seq).or_default()
    if (pos != s.len)
      return fail(LTKV_ERR_NONCONTIG, "seq %u: position %zu is not contiguous (length %zu)", seq,
                  pos, s.len);
    const size_t sl = pos % LTKV_BLOCK;
    if (sl == 0) {
      int32_t b;
      if (!alloc(&b)) return fail(LTKV_ERR_FULL, "KV cache full");
      s.blocks.push_back(b);
      rt_mark(seq, s.blocks.size() - 1, s.blocks.size());
    } else {
      const int32_t last = s.blocks.back();
      if (refs[last] > 1) {  // the sequence diverges from a shared prefix
        int32_t nb;
        if (!alloc(&nb)) return fail(LTKV_ERR_FULL, "KV cache full");
        pending.push_back(last);
        pending.push_back(nb);
        release(last);
        s.blocks.back() = nb;
        rt_mark(seq, s.blocks.size() - 1, s.blocks.size());
        ++cow_copies;
      }
    }
    s.len = pos + 1;
    *block = (uint32_t)s.blocks.back();
    *slot = (uint32_t)sl;
    return LTKV_OK;
  }

  // Enqueue the pending copy-on-write copies (kernel 2) on the stream.
  int flush_pending() {
    if (pending.empty()) return LTKV_OK;
    if (device == LTKV_NO_DEVICE) {  // no pools: only the metadata changes
      pending.clear();
      return LTKV_OK;
    }
    const size_t n = pending.size() / 2;
    DeviceGuard dg(device);
    if (!dg.ok) return fail(LTKV_ERR_HIP, "hipSetDevice(%d) failed", device);
    if (pairs_in_flight) {  // the staging buffer may still be read by the last copy
      HIP_TRY(hipEventSynchronize(pairs_done), "hipEventSynchronize");
      pairs_in_flight = false;
    }
    if (n > pairs_cap) {
      size_t cap = std::max<size_t>(n, 2 * pairs_cap);
      cap = std::max<size_t>(cap, 256);
      if (d_pairs) {  // the last copy kernel may still read the old device pairs
        HIP_TRY(stream ? hipStreamSynchronize(stream) : hipDeviceSynchronize(), "synchronize");
        (void)hipFree(d_pairs);
      }
      if (h_pairs) (void)hipHostFree(h_pairs);
      h_pairs = nullptr;
      d_pairs = nullptr;
      pairs_cap = 0;
      HIP_TRY(hipHostMalloc((void **)&h_pairs, cap * 2 * sizeof(int32_t), hipHostMallocDefault),
              "hipHostMalloc(copy pairs)");
      HIP_TRY(hipMalloc((void **)&d_pairs, cap * 2 * sizeof(int32_t)), "hipMalloc(copy pairs)");
      pairs_cap = cap;
    }
    // Ascending destination order: the copies of a batch are independent
    // (every destination is a fresh block, no source is freed within the
    // batch), and destination-ordered writes are faster on this part.
    std::vector<std::pair<int32_t, int32_t>> &pv = pending_sorted;
    pv.resize(n);
    for (size_t i = 0; i < n; ++i) pv[i] = {pending[2 * i + 1], pending[2 * i]};
    std::sort(pv.begin(), pv.end());
    for (size_t i = 0; i < n; ++i) {
      h_pairs[2 * i] = pv[i].second;
      h_pairs[2 * i + 1] = pv[i].first;
    }
    pending.clear();
    HIP_TRY(hipMemcpyAsync(d_pairs, h_pairs, n * 2 * sizeof(int32_t), hipMemcpyHostToDevice, stream),
            "hipMemcpyAsync(copy pairs)");
    HIP_TRY(hipEventRecord(pairs_done, stream), "hipEventRecord");
    pairs_in_flight = true;
    const bool bulk = n >= kCopyOrderMinPairs;
    HIP_TRY(ltkv::launch_copy_blocks(geom, (int)n_layers, k, v, d_pairs, (int64_t)n, bulk, stream),
            "copy_blocks launch");
    if (q8())
      HIP_TRY(ltkv::launch_copy_blocks(sgeom, (int)n_layers, ks, vs, d_pairs, (int64_t)n, bulk, stream),
              "copy_blocks launch (scales)");
    return LTKV_OK;
  }

  void truncate(uint32_t seq, size_t from) {  // kv.rs:153-169
    ++gen;
    auto it = seqs.find(seq);
    if (it == seqs.end()) return;
    Seq &s = it->second;
    if (from >= s.len) return;
    const size_t keep = (from + LTKV_BLOCK - 1) / LTKV_BLOCK;
    for (size_t i = keep; i < s.blocks.size(); ++i) release(s.blocks[i]);
    s.blocks.resize(keep);
    s.len = from;
    if (from == 0) {
      seqs.erase(it);
      rt_remove(seq);
    } else {
      rt_mark(seq, 0, 0);  // the table length changed
    }
  }

  void share(uint32_t src, uint32_t dst, size_t len) {  // kv.rs:172-183
    ++gen;
    truncate(dst, 0);
    auto it = seqs.find(src);
    if (it == seqs.end()) return;
    len = std::min(len, it->second.len);
    const size_t nb = (len + LTKV_BLOCK - 1) / LTKV_BLOCK;
    std::vector<int32_t> blocks(it->second.blocks.begin(), it->second.blocks.begin() + nb);
    for (int32_t b : blocks) refs[b] += 1;
    if (len > 0) {
      seqs[dst] = Seq{std::move(blocks), len};
      rt_mark(dst, 0, nb);
    }
  }
};

namespace {

// Takes the device ops' fault word in stream order (after everything enqueued
// before it on the cache's stream): one kernel swaps it to zero on the device,
// then the taken value is read back. LTKV_OK, or the first fault as
// LTKV_ERR_RANGE / LTKV_ERR_ARG.
int take_status(ltkv_cache *c) {
  HIP_TRY(ltkv::launch_status_take(c->d_status, c->stream), "status launch");
  int32_t st[2] = {0, 0};
  HIP_TRY(hipMemcpyAsync(st, c->d_status + 2, sizeof st, hipMemcpyDeviceToHost, c->stream),
          "hipMemcpyAsync(status)");
  HIP_TRY(c->stream ? hipStreamSynchronize(c->stream) : hipDeviceSynchronize(), "synchronize");
  if (st[0] == 0) return LTKV_OK;
  if (st[0] & 1)  // kv.rs:147 panics on such an index
    return fail(LTKV_ERR_RANGE,
                "a device op read a block-table entry outside the pool (query or sequence %d); it read "
                "block 0 in its place (attention) or copied nothing (gather)",
                st[1]);
  return fail(LTKV_ERR_ARG,
              "fused append + attention: the cell of query %d is not position len - 1 of its table", st[1]);
}

int check_attention_shape(const ltkv_cache *c, size_t n_heads, size_t head_dim, size_t *group) {
  if (head_dim == 0 || c->kv_dim % head_dim != 0)
    return fail(LTKV_ERR_ARG, "head_dim %zu does not divide kv_dim %zu", head_dim, c->kv_dim);
  const size_t n_kv_heads = c->kv_dim / head_dim;
  if (n_heads == 0 || n_heads % n_kv_heads != 0)
    return fail(LTKV_ERR_ARG, "n_heads %zu is not a multiple of n_kv_heads %zu", n_heads, n_kv_heads);
  *group = n_heads / n_kv_heads;
  if (!ltkv::attention_supported((int)c->elem, (int)head_dim, (int)*group))
    return fail(LTKV_ERR_ARG, "unsupported shape: head_dim %zu (at most 1024), group %zu", head_dim, *group);
  return LTKV_OK;
}

// Grows the attention workspace to at least `bytes` (device of the cache current).
int ensure_workspace(ltkv_cache *c, size_t bytes) {
  if (bytes <= c->ws_bytes) return LTKV_OK;
  if (c->ws) {
    // The old workspace may still be read by enqueued work.
    HIP_TRY(c->stream ? hipStreamSynchronize(c->stream) : hipDeviceSynchronize(), "synchronize");
    HIP_TRY(hipFree(c->ws), "hipFree(workspace)");
    c->ws = nullptr;
    c->ws_bytes = 0;
  }
  HIP_TRY(hipMalloc((void **)&c->ws, bytes), "hipMalloc(workspace)");
  c->ws_bytes = bytes;
  return LTKV_OK;
}

// Uploads the resident-table changes made since the last call: only the
// changed entries of changed rows, as (row, col, value) triples through
// pinned staging, applied by one small kernel on the cache stream. Growing
// the tables (more rows, or a table longer than the width) reallocates them
// and uploads every live row once. Device of the cache current.
int sync_tables(ltkv_cache *c) {
  const size_t need_rows = c->rt_seq.size();
  size_t need_w = c->rt_width;
  // Blocks of the live sequence in row r (0 for a free row).
  auto row_blocks = [&](int32_t r) -> const std::vector<int32_t> * {
    if (!c->rt_live[r]) return nullptr;
    const auto it = c->seqs.find(c->rt_seq[r]);
    return it == c->seqs.end() ? nullptr : &it->second.blocks;
  };
  for (int32_t r : c->rt_dirty_rows)
    if (const std::vector<int32_t> *b = row_blocks(r)) need_w = std::max(need_w, b->size());
  const bool grow = !c->d_rt || need_rows > c->rt_rows || need_w > c->rt_width;
  if (!grow && c->rt_dirty_rows.empty()) return LTKV_OK;
  std::vector<int32_t> &u = c->rt_upd;
  u.clear();
  auto row_updates = [&](int32_t r, size_t lo, size_t hi) {
    const std::vector<int32_t> *b = row_blocks(r);
    if ((size_t)r < c->rt_nb.size()) c->rt_nb[r] = b ? (uint32_t)b->size() : 0;
    if (!b) {  // released: an empty table
      u.insert(u.end(), {r, -1, 0});
      return;
    }
    const std::vector<int32_t> &blocks = *b;
    hi = std::min(hi, blocks.size());
    for (size_t j = lo; j < hi; ++j) u.insert(u.end(), {r, (int32_t)j, blocks[j]});
    u.insert(u.end(), {r, -1, (int32_t)blocks.size()});
  };
  if (grow) {
    const size_t rows = std::max<size_t>({need_rows, 2 * c->rt_rows, 64});
    const size_t width = std::max<size_t>({need_w, 2 * c->rt_width, 64});
    if ((uint64_t)rows * width > (uint64_t)INT32_MAX)
      return fail(LTKV_ERR_ARG, "resident block tables too large (%zu rows x %zu blocks)", rows, width);
    // The old tables may still be read by enqueued work.
    HIP_TRY(c->stream ? hipStreamSynchronize(c->stream) : hipDeviceSynchronize(), "synchronize");
    if (c->d_rt) (void)hipFree(c->d_rt);
    if (c->d_rt_nb) (void)hipFree(c->d_rt_nb);
    c->d_rt = c->d_rt_nb = nullptr;
    c->rt_rows = c->rt_width = 0;
    HIP_TRY(hipMalloc((void **)&c->d_rt, rows * width * sizeof(int32_t)), "hipMalloc(resident tables)");
    HIP_TRY(hipMalloc((void **)&c->d_rt_nb, rows * sizeof(int32_t)), "hipMalloc(resident table lengths)");
    c->rt_rows = rows;
    c->rt_width = width;
    for (size_t r = 0; r < rows; ++r) {
      if (r < need_rows) row_updates((int32_t)r, 0, SIZE_MAX);
      else u.insert(u.end(), {(int32_t)r, -1, 0});
    }
  } else {
    for (int32_t r : c->rt_dirty_rows) row_updates(r, c->rt_lo[r], c->rt_hi[r]);
  }
  for (int32_t r : c->rt_dirty_rows) c->rt_dirty[r] = 0;
  c->rt_dirty_rows.clear();

  const size_t n = u.size() / 3;
  if (n <= (size_t)ltkv::kTableUpdateArgs) {
    // A step's few changes (new blocks, copy-on-write replacements, lengths)
    // travel in the update kernel's arguments: no staging copy, no event.
    ltkv::TableUpdates args;
    args.n = (int32_t)n;
    std::memcpy(args.t, u.data(), n * 3 * sizeof(int32_t));
    HIP_TRY(ltkv::launch_table_update_args(c->d_rt, c->d_rt_nb, (int64_t)c->rt_width, (int64_t)c->rt_rows, args,
                                           c->stream),
            "table update launch");
    c->rt_uploaded += n;
    return LTKV_OK;
  }
  if (c->rt_in_flight) {  // the staging buffer may still be read by the last upload
    HIP_TRY(hipEventSynchronize(c->rt_done), "hipEventSynchronize");
    c->rt_in_flight = false;
  }
  if (n > c->rt_upd_cap) {
    const size_t cap = std::max<size_t>({n, 2 * c->rt_upd_cap, 1024});
    if (c->h_rt_upd) (void)hipHostFree(c->h_rt_upd);
    if (c->d_rt_upd) {
      HIP_TRY(c->stream ? hipStreamSynchronize(c->stream) : hipDeviceSynchronize(), "synchronize");
      (void)hipFree(c->d_rt_upd);
    }
    c->h_rt_upd = c->d_rt_upd = nullptr;
    c->rt_upd_cap = 0;
    HIP_TRY(hipHostMalloc((void **)&c->h_rt_upd, cap * 3 * sizeof(int32_t), hipHostMallocDefault),
            "hipHostMalloc(table updates)");
    HIP_TRY(hipMalloc((void **)&c->d_rt_upd, cap * 3 * sizeof(int32_t)), "hipMalloc(table updates)");
    c->rt_upd_cap = cap;
  }
  std::memcpy(c->h_rt_upd, u.data(), n * 3 * sizeof(int32_t));
  HIP_TRY(hipMemcpyAsync(c->d_rt_upd, c->h_rt_upd, n * 3 * sizeof(int32_t), hipMemcpyHostToDevice,
                         c->stream),
          "hipMemcpyAsync(table updates)");
  HIP_TRY(hipEventRecord(c->rt_done, c->stream), "hipEventRecord");
  c->rt_in_flight = true;
  HIP_TRY(ltkv::launch_table_update(c->d_rt, c->d_rt_nb, (int64_t)c->rt_width, (int64_t)c->rt_rows,
                                    c->d_rt_upd, (int64_t)n, c->stream),
          "table update launch");
  c->rt_uploaded += n;
  return LTKV_OK;
}

// Longest table (blocks) of a live sequence.
// Longest resident table (blocks), as of the last sync_tables.
size_t max_table_blocks(const ltkv_cache *c) {
  uint32_t m = 0;
  for (uint32_t nb : c->rt_nb) m = std::max(m, nb);
  return m;
}

ltkv::PoolGeom head_geom(const ltkv_cache *c, size_t head_dim) {
  ltkv::PoolGeom g = c->geom;
  g.head_stride = (int64_t)head_dim;  // token-major: heads are adjacent in a row
  return g;
}

ltkv::AttnArgs attn_args(ltkv_cache *c, size_t layer, size_t n, size_t n_heads, size_t head_dim,
                         float scale, const float *d_q, float *d_out, const ltkv::AttnWorkspace &ws,
                         int part, int max_parts, uint8_t *ws_base) {
  ltkv::AttnArgs a{};
  a.k_layer = c->k_layer(layer);
  a.v_layer = c->v_layer(layer);
  a.k_scale = c->k_scales(layer);
  a.v_scale = c->v_scales(layer);
  a.q = d_q;
  a.out = d_out;
  a.part_o = ws.bytes ? (float *)(ws_base + ws.part_o_off) : nullptr;
  a.part_ml = ws.bytes ? (float *)(ws_base + ws.part_ml_off) : nullptr;
  a.n = (int64_t)n;
  a.n_heads = (int)n_heads;
  a.n_kv_heads = (int)(c->kv_dim / head_dim);
  a.head_dim = (int)head_dim;
  a.scale = scale;
  a.part_tokens = part;
  a.max_parts = max_parts;
  a.split = 1;
  a.valu = c->attn_engine == LTKV_ENGINE_VALU && c->elem == 2;
  a.status = c->d_status;
  a.cu_count = c->device_count_cu;
  return a;
}

// Fewest shared full blocks and members for a prefix group.
constexpr size_t kMinSharedBlocks = 2;
// Tokens per group partition are at least this (a multiple of the kernel's
// 32-token staging step).
constexpr size_t kMinPrefixPart = 256;
// Longest per-query remainder for which grouped plans size the per-query pass's items themselves.
constexpr size_t kShortRemainder = 512;

size_t align8(size_t x) { return (x + 7) / 8 * 8; }

// Orders group jobs by work-group id. Work-group b runs on XCD b % 8 (each
// XCD has its own L2): the jobs of one K/V range (adjacent in `jobs`, same
// token range and kv head, different member tiles) go to one XCD, ranges are
// spread over the XCDs longest first onto the least loaded one, and each
// XCD runs its longest jobs first. Empty jobs pad the XCD queues.
std::vector<ltkv::MqJob> place_jobs(const std::vector<ltkv::MqJob> &jobs) {
  constexpr int kXcds = 8;
  struct Range {
    size_t first, count;
    uint64_t work;
  };
  std::vector<Range> ranges;
  for (size_t i = 0; i < jobs.size(); ++i) {
    const ltkv::MqJob &j = jobs[i];
    const uint64_t w = (uint64_t)(j.t1 - j.t0);
    if (!ranges.empty()) {
      const ltkv::MqJob &f = jobs[ranges.back().first];
      if (f.table == j.table && f.t0 == j.t0 && f.kvh == j.kvh) {
        ranges.back().count++;
        ranges.back().work += w;
        continue;
      }
    }
    ranges.push_back({i, 1, w});
  }
  std::stable_sort(ranges.begin(), ranges.end(), [](const Range &a, const Range &b) { return a.work > b.work; });
  std::vector<std::vector<ltkv::MqJob>> queue(kXcds);
  std::vector<uint64_t> load(kXcds, 0);
  for (const Range &r : ranges) {
    const int x = (int)(std::min_element(load.begin(), load.end()) - load.begin());
    for (size_t k = 0; k < r.count; ++k) queue[x].push_back(jobs[r.first + k]);
    load[x] += r.work;
  }
  size_t depth = 0;
  for (auto &q : queue) {
    std::stable_sort(q.begin(), q.end(),
                     [](const ltkv::MqJob &a, const ltkv::MqJob &b) { return a.t1 - a.t0 > b.t1 - b.t0; });
    depth = std::max(depth, q.size());
  }
  std::vector<ltkv::MqJob> out(depth * kXcds);  // zero-initialised: empty jobs
  for (int x = 0; x < kXcds; ++x)
    for (size_t k = 0; k < queue[x].size(); ++k) out[k * kXcds + x] = queue[x][k];
  return out;
}

// Builds the plan's host arrays: tables, prefix groups, suffix tables, jobs.
int build_plan(ltkv_cache *c, size_t n, const uint32_t *seqs, const uint32_t *lens, size_t n_heads,
               size_t head_dim, size_t group, unsigned flags) {
  AttnPlan &P = c->plan;
  std::vector<const Seq *> sq(n, nullptr);
  size_t stride = 1;
  for (size_t i = 0; i < n; ++i) {
    auto it = c->seqs.find(seqs[i]);
    const size_t have = it == c->seqs.end() ? 0 : it->second.len;
    if (lens[i] > have)
      return fail(LTKV_ERR_RANGE, "query %zu: length %u exceeds the %zu tokens of seq %u", i, lens[i],
                  have, seqs[i]);
    if (it != c->seqs.end()) sq[i] = &it->second;
    stride = std::max<size_t>(stride, (lens[i] + LTKV_BLOCK - 1) / LTKV_BLOCK);
  }

  // Groups whose rows attend to a common token range [0, tokens) of one
  // block table together, each row up to its own limit:
  //  * causal groups: several queries of one sequence (the tokens of a
  //    prefill chunk); the range is the longest query's context and each
  //    query is masked at its own length (model.rs:435-475 over all tokens);
  //  * prefix groups: the rest, bucketed by first block; in a bucket, the
  //    member set and shared length (common leading full blocks) that save
  //    the most block reads, (members - 1) * blocks; each member reads the
  //    rest of its context in the per-query pass.
  struct Group {
    std::vector<int32_t> members;
    size_t tokens;
    int32_t table_query;  // a member whose table covers the range
  };
  std::vector<Group> groups;
  std::vector<size_t> pre_tokens(n, 0);  // context of query i covered by its group
  const size_t n_kv_heads = c->kv_dim / head_dim;
  // Groups need the shared-prefix kernel and a per-query pass that folds
  // their partials (the tuned decode kernels); other shapes plan per query.
  if ((flags & LTKV_PLAN_SHARED_PREFIX) && ltkv::mq_supported((int)c->elem, (int)head_dim, (int)group) &&
      ltkv::attention_tuned((int)c->elem, (int)head_dim, (int)group)) {
    std::vector<char> taken(n, 0);
    {
      // Queries of one sequence (in query order), sequences in the order of
      // their first query. A batch's queries of one sequence usually come in
      // one run (a prefill chunk), so the runs of equal sequences are sorted,
      // not the queries (a sort of (sequence, query) pairs took ~200 us of a
      // 4096-token plan), and only sequences with two queries or more get a
      // member list.
      std::vector<std::pair<size_t, size_t>> runs;  // [start, end) of equal sequences
      for (size_t i = 0; i < n;) {
        size_t e = i + 1;
        while (e < n && seqs[e] == seqs[i]) ++e;
        runs.emplace_back(i, e);
        i = e;
      }
      std::vector<std::pair<uint32_t, uint32_t>> by_run;  // (sequence, run)
      by_run.reserve(runs.size());
      for (size_t r = 0; r < runs.size(); ++r) by_run.emplace_back(seqs[runs[r].first], (uint32_t)r);
      std::sort(by_run.begin(), by_run.end());
      std::vector<std::vector<int32_t>> by_seq;
      for (size_t a = 0; a < by_run.size();) {
        size_t e = a + 1, count = 0;
        while (e < by_run.size() && by_run[e].first == by_run[a].first) ++e;
        for (size_t k = a; k < e; ++k)
          for (size_t i = runs[by_run[k].second].first; i < runs[by_run[k].second].second; ++i) count += lens[i] > 0;
        if (count >= 2) {
          by_seq.emplace_back();
          by_seq.back().reserve(count);
          for (size_t k = a; k < e; ++k)  // runs in query order (sorted by run index)
            for (size_t i = runs[by_run[k].second].first; i < runs[by_run[k].second].second; ++i)
              if (lens[i] > 0) by_seq.back().push_back((int32_t)i);
        }
        a = e;
      }
      std::sort(by_seq.begin(), by_seq.end(),
                [](const std::vector<int32_t> &x, const std::vector<int32_t> &y) { return x[0] < y[0]; });
      for (auto &b : by_seq) {
        if (b.size() < 2) continue;
        Group gr;
        gr.table_query = b[0];
        for (int32_t m : b)
          if (lens[m] > lens[gr.table_query]) gr.table_query = m;
        gr.tokens = lens[gr.table_query];
        if (gr.tokens < kMinSharedBlocks * LTKV_BLOCK) continue;
        if (!std::is_sorted(b.begin(), b.end(), [&](int32_t x, int32_t y) { return lens[x] < lens[y]; }))
          std::stable_sort(b.begin(), b.end(), [&](int32_t x, int32_t y) { return lens[x] < lens[y]; });
        gr.members = b;
        for (int32_t m : b) {
          taken[m] = 1;
          pre_tokens[m] = lens[m];
        }
        groups.push_back(std::move(gr));
      }
    }
    std::unordered_map<int32_t, size_t> bucket_of;
    std::vector<std::vector<int32_t>> buckets;
    for (size_t i = 0; i < n; ++i) {
      if (taken[i] || lens[i] / LTKV_BLOCK < kMinSharedBlocks) continue;
      auto ins = bucket_of.emplace(sq[i]->blocks[0], buckets.size());
      if (ins.second) buckets.emplace_back();
      buckets[ins.first->second].push_back((int32_t)i);
    }
    for (const auto &b : buckets) {
      if (b.size() < 2) continue;
      const std::vector<int32_t> &ref = sq[b[0]]->blocks;
      const size_t ref_full = lens[b[0]] / LTKV_BLOCK;
      std::vector<std::pair<size_t, int32_t>> lcp;  // (shared full blocks with b[0], query)
      lcp.reserve(b.size());
      for (int32_t m : b) {
        const size_t cap = std::min<size_t>(lens[m] / LTKV_BLOCK, ref_full);
        const int32_t *x = sq[m]->blocks.data(), *y = ref.data();
        size_t k = 0;
        while (k + 16 <= cap && std::memcmp(x + k, y + k, 16 * sizeof(int32_t)) == 0) k += 16;
        while (k < cap && x[k] == y[k]) ++k;
        lcp.emplace_back(k, m);
      }
      std::stable_sort(lcp.begin(), lcp.end(),
                       [](const auto &x, const auto &y) { return x.first > y.first; });
      size_t best = 0, best_count = 0;
      for (size_t cnt = 2; cnt <= lcp.size(); ++cnt) {
        const size_t blocks = lcp[cnt - 1].first;
        if (blocks < kMinSharedBlocks) break;
        if ((cnt - 1) * blocks > best) {
          best = (cnt - 1) * blocks;
          best_count = cnt;
        }
      }
      if (best_count < 2) continue;
      Group gr;
      gr.tokens = lcp[best_count - 1].first * LTKV_BLOCK;
      for (size_t k = 0; k < best_count; ++k) gr.members.push_back(lcp[k].second);
      std::sort(gr.members.begin(), gr.members.end());
      gr.table_query = gr.members[0];
      for (int32_t m : gr.members) pre_tokens[m] = gr.tokens;
      groups.push_back(std::move(gr));
    }
  }

  // Group jobs: member tiles of mq_rows query rows; each group's range is
  // split into partitions so the launch has about two waves per SIMD. A job
  // is skipped when every row of its tile ends before its partition starts;
  // a member has partials for the partitions that start below its limit.
  // With one partition, a tile whose members read nothing else writes their
  // outputs itself (pre_parts -1: no per-query pass, no merge).
  const size_t per_job = (size_t)ltkv::mq_rows((int)c->elem, (int)head_dim) / group;  // members per work-group
  size_t units = 0;
  for (const auto &gr : groups) units += (gr.members.size() + per_job - 1) / per_job * n_kv_heads;
  const size_t waves = (size_t)ltkv::mq_rows((int)c->elem, (int)head_dim) / 32;
  const size_t target = 8 * (size_t)c->device_count_cu / waves;  // two waves per SIMD
  // Work-groups run one per CU and take their jobs longest first, so no job
  // should be longer than the average load of one: a group whose range is
  // longer than the mean tokens per work-group slot is cut into ranges of
  // about that length (prefill 8 x 512 at contexts up to 7k: the longest
  // chunk's jobs alone set the kernel's end, 19% past the mean load).
  size_t work = 0;  // token-rows of all jobs, counted as full ranges
  for (const auto &gr : groups) work += (gr.members.size() + per_job - 1) / per_job * n_kv_heads * gr.tokens;
  const size_t mean_tokens = std::max<size_t>(1, work / std::max<size_t>(1, target));
  std::vector<ltkv::MqJob> jobs;
  std::vector<int32_t> members;
  std::vector<int32_t> pre_parts(n, 0);
  int max_pre_parts = 0;
  uint64_t shared_blocks = 0, grouped = 0;
  size_t gstride = 1;
  for (const auto &gr : groups) gstride = std::max<size_t>(gstride, (gr.tokens + LTKV_BLOCK - 1) / LTKV_BLOCK);
  for (size_t gi = 0; gi < groups.size(); ++gi) {
    const Group &gr = groups[gi];
    const size_t tokens = gr.tokens;
    const size_t max_split = std::max<size_t>(1, tokens / kMinPrefixPart);
    const size_t fill = std::max<size_t>((target + units - 1) / units, (tokens + mean_tokens - 1) / mean_tokens);
    const size_t split = std::max(std::min(max_split, std::max<size_t>(1, fill)),
                                  (tokens + ltkv::kMqMaxRange - 1) / ltkv::kMqMaxRange);
    const size_t pt = ((tokens + split - 1) / split + 31) / 32 * 32;
    const size_t parts = (tokens + pt - 1) / pt;
    const size_t m0 = members.size() / 2;
    for (int32_t m : gr.members) {
      const size_t limit = std::min<size_t>(lens[m], tokens);
      members.push_back(m);
      members.push_back((int32_t)limit);
      pre_parts[m] = (int32_t)((limit + pt - 1) / pt);
    }
    const size_t tiles = (gr.members.size() + per_job - 1) / per_job;
    std::vector<char> direct(tiles, 0);
    if (parts == 1) {
      for (size_t t = 0; t < tiles; ++t) {
        const size_t first = t * per_job, count = std::min(per_job, gr.members.size() - first);
        bool alone = true;
        for (size_t k = first; k < first + count; ++k)
          alone = alone && pre_tokens[gr.members[k]] >= lens[gr.members[k]];
        direct[t] = alone;
        if (alone)
          for (size_t k = first; k < first + count; ++k) pre_parts[gr.members[k]] = -1;
      }
    }
    for (size_t p = 0; p < parts; ++p)
      for (size_t h = 0; h < n_kv_heads; ++h)
        for (size_t t = 0; t < tiles; ++t) {
          const size_t first = t * per_job, count = std::min(per_job, gr.members.size() - first);
          size_t top = 0;  // highest limit in the tile
          for (size_t k = first; k < first + count; ++k)
            top = std::max<size_t>(top, members[2 * (m0 + k) + 1]);
          if (top <= p * pt) continue;
          ltkv::MqJob j{};
          j.table = (int32_t)(gi * gstride);
          j.t0 = (int32_t)(p * pt);
          j.t1 = (int32_t)std::min(std::min(tokens, (p + 1) * pt), top);
          j.member0 = (int32_t)(m0 + first);
          j.n_members = (int32_t)count;
          j.part = (int32_t)p;
          j.kvh = (int32_t)h;
          j.direct = direct[t];
          jobs.push_back(j);
        }
    max_pre_parts = std::max(max_pre_parts, (int)parts);
    shared_blocks += (tokens + LTKV_BLOCK - 1) / LTKV_BLOCK;
    grouped += gr.members.size();
  }
  jobs = place_jobs(jobs);

  size_t sstride = 1;
  uint64_t suffix_tokens = 0;
  // The per-query pass reads positions [pre_tokens, len): whole blocks after a
  // prefix group's range, nothing after a causal group's.
  std::vector<size_t> pre_blocks(n, 0);
  for (size_t i = 0; i < n; ++i) {
    const size_t nb = (lens[i] + LTKV_BLOCK - 1) / LTKV_BLOCK;
    pre_blocks[i] = pre_tokens[i] >= lens[i] ? nb : pre_tokens[i] / LTKV_BLOCK;
    sstride = std::max<size_t>(sstride, nb - pre_blocks[i]);
    suffix_tokens += lens[i] - pre_tokens[i];
  }
  // With groups the per-query pass covers the (usually short) remainders:
  // one wave per item, about eight items per CU, whatever the batch.
  const uint64_t per_wg = suffix_tokens * n_kv_heads / (8 * (uint64_t)c->device_count_cu) + 1;
  P.suffix_part = (int)std::min<uint64_t>(1024, std::max<uint64_t>(64, (per_wg + 63) / 64 * 64));
  if ((uint64_t)n * sstride + (uint64_t)groups.size() * gstride > (uint64_t)INT32_MAX / 2)
    return fail(LTKV_ERR_ARG, "block tables of this batch are too large");
  std::vector<int32_t> qmap;  // queries left for the per-query pass
  size_t max_suffix = 0;
  bool empty_with_groups = false, pass_empty = true;
  for (size_t i = 0; i < n; ++i)
    if (pre_parts[i] >= 0) {
      qmap.push_back((int32_t)i);
      const size_t rem = lens[i] > pre_tokens[i] ? lens[i] - pre_tokens[i] : 0;
      max_suffix = std::max(max_suffix, rem);
      if (pre_parts[i] > 0 && rem == 0) empty_with_groups = true;
      if (pre_parts[i] == 0 || rem > 0) pass_empty = false;
    }
  const bool groups_only = qmap.empty();

  P.n = n;
  P.n_heads = n_heads;
  P.head_dim = head_dim;
  P.stride = stride;
  P.sstride = sstride;
  P.max_pre_parts = max_pre_parts;
  P.n_jobs = (int)jobs.size();
  P.groups = groups.size();
  P.grouped = grouped;
  P.shared_blocks = shared_blocks;
  P.groups_only = groups_only;
  P.n_pass = qmap.size();
  P.max_suffix = max_suffix;
  P.empty_with_groups = empty_with_groups;
  P.pass_empty = pass_empty && !groups_only;
  P.off_tables = 0;
  P.off_stables = align8(P.off_tables + groups.size() * gstride);
  P.off_slens = align8(P.off_stables + n * sstride);
  P.off_pre = align8(P.off_slens + n);
  P.off_qmap = align8(P.off_pre + n);
  P.off_members = align8(P.off_qmap + qmap.size());
  P.off_jobs = align8(P.off_members + members.size());
  const size_t words = P.off_jobs + jobs.size() * (sizeof(ltkv::MqJob) / 4);
  P.bytes = words * 4;
  P.host.assign(words, 0);
  int32_t *h = P.host.data();
  for (size_t gi = 0; gi < groups.size(); ++gi) {
    const std::vector<int32_t> &blocks = sq[groups[gi].table_query]->blocks;
    const size_t nb = (groups[gi].tokens + LTKV_BLOCK - 1) / LTKV_BLOCK;
    int32_t *row = h + P.off_tables + gi * gstride;
    for (size_t k = 0; k < gstride; ++k) row[k] = k < nb ? blocks[k] : -1;
  }
  for (size_t i = 0; i < n; ++i) {
    const size_t nb = (lens[i] + LTKV_BLOCK - 1) / LTKV_BLOCK;
    int32_t *srow = h + P.off_stables + i * sstride;
    for (size_t k = 0; k < sstride; ++k) srow[k] = pre_blocks[i] + k < nb ? sq[i]->blocks[pre_blocks[i] + k] : -1;
    h[P.off_slens + i] = (int32_t)(lens[i] - pre_tokens[i]);
    h[P.off_pre + i] = pre_parts[i];
  }
  std::copy(qmap.begin(), qmap.end(), h + P.off_qmap);
  std::copy(members.begin(), members.end(), h + P.off_members);
  if (!jobs.empty()) std::memcpy(h + P.off_jobs, jobs.data(), jobs.size() * sizeof(ltkv::MqJob));
  return LTKV_OK;
}

// Copies the plan's arrays to the device on the cache stream (pinned staging).
int upload_plan(ltkv_cache *c) {
  AttnPlan &P = c->plan;
  DeviceGuard dg(c->device);
  if (!dg.ok) return fail(LTKV_ERR_HIP, "hipSetDevice(%d) failed", c->device);
  if (!P.done) HIP_TRY(hipEventCreateWithFlags(&P.done, hipEventDisableTiming), "hipEventCreate");
  if (P.in_flight) {  // the staging buffer may still be read by the last upload
    HIP_TRY(hipEventSynchronize(P.done), "hipEventSynchronize");
    P.in_flight = false;
  }
  if (P.bytes > P.cap) {
    const size_t cap = std::max<size_t>(P.bytes, 2 * P.cap);
    if (P.d) {  // enqueued attention may still read the old tables
      HIP_TRY(c->stream ? hipStreamSynchronize(c->stream) : hipDeviceSynchronize(), "synchronize");
      HIP_TRY(hipFree(P.d), "hipFree(plan)");
      P.d = nullptr;
    }
    if (P.h) (void)hipHostFree(P.h);
    P.h = nullptr;
    P.cap = 0;
    HIP_TRY(hipHostMalloc((void **)&P.h, cap, hipHostMallocDefault), "hipHostMalloc(plan)");
    HIP_TRY(hipMalloc((void **)&P.d, cap), "hipMalloc(plan)");
    P.cap = cap;
  }
  std::memcpy(P.h, P.host.data(), P.bytes);
  HIP_TRY(hipMemcpyAsync(P.d, P.h, P.bytes, hipMemcpyHostToDevice, c->stream), "hipMemcpyAsync(plan)");
  HIP_TRY(hipEventRecord(P.done, c->stream), "hipEventRecord");
  P.in_flight = true;
  return LTKV_OK;
}

}  // namespace

extern "C" {

const char *ltkv_last_error(void) { return g_err; }

int ltkv_create(size_t n_layers, size_t kv_dim, size_t n_tokens, int dtype, int device,
                ltkv_cache **out) {
  if (!out) return fail(LTKV_ERR_ARG, "out is null");
  *out = nullptr;
  if (n_layers == 0 || kv_dim == 0) return fail(LTKV_ERR_ARG, "n_layers and kv_dim must be > 0");
  if (dtype != LTKV_F16 && dtype != LTKV_F32 && dtype != LTKV_Q8_0)
    return fail(LTKV_ERR_ARG, "dtype must be F16, F32 or Q8_0");
  if (dtype == LTKV_Q8_0 && kv_dim % 32 != 0)
    return fail(LTKV_ERR_ARG, "Q8_0 needs kv_dim a multiple of 32 (one scale per 32 elements)");
  const size_t n_blocks = (n_tokens + LTKV_BLOCK - 1) / LTKV_BLOCK;  // kv.rs:36
  if (n_blocks > (size_t)INT32_MAX / LTKV_BLOCK)
    return fail(LTKV_ERR_ARG, "n_tokens too large for 32-bit cell indices");
  if (device != LTKV_NO_DEVICE) {
    int ndev = 0;
    HIP_TRY(hipGetDeviceCount(&ndev), "hipGetDeviceCount");
    if (device < 0 || device >= ndev)
      return fail(LTKV_ERR_ARG, "device %d out of range (%d HIP devices)", device, ndev);
  }

  ltkv_cache *c = new (std::nothrow) ltkv_cache();
  if (!c) return fail(LTKV_ERR_ARG, "out of host memory");
  c->device = device;
  c->dtype = dtype;
  c->n_layers = n_layers;
  c->kv_dim = kv_dim;
  c->n_blocks = n_blocks;
  c->elem = dtype == LTKV_F16 ? 2 : dtype == LTKV_F32 ? 4 : 1;
  c->geom.n_blocks = (int64_t)n_blocks;
  c->geom.block_stride = (int64_t)(LTKV_BLOCK * kv_dim);
  c->geom.slot_stride = (int64_t)kv_dim;
  c->geom.head_stride = 0;  // token-major: set per call from head_dim
  c->geom.kv_dim = (int)kv_dim;
  c->geom.elem = (int)c->elem;
  c->sgeom = c->geom;
  c->sgeom.block_stride = (int64_t)(LTKV_BLOCK * (kv_dim / 32));
  c->sgeom.slot_stride = (int64_t)(kv_dim / 32);
  c->sgeom.kv_dim = (int)(kv_dim / 32);
  c->sgeom.elem = 2;
  c->refs.assign(n_blocks, 0);
  c->free.reserve(n_blocks);
  for (size_t b = n_blocks; b-- > 0;) c->free.push_back((int32_t)b);  // (0..n).rev()

  if (device == LTKV_NO_DEVICE) {
    *out = c;
    return LTKV_OK;
  }
  DeviceGuard dg(device);
  if (!dg.ok) {
    delete c;
    return fail(LTKV_ERR_HIP, "hipSetDevice(%d) failed", device);
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) == hipSuccess && prop.multiProcessorCount > 0)
    c->device_count_cu = prop.multiProcessorCount;
  {
    void *p = nullptr;
    const hipError_t e = ltkv::scratch_address(device, &p);
    if (e != hipSuccess) {
      delete c;
      return hip_fail(e, "hipGetSymbolAddress(scratch)");
    }
    c->scratch = static_cast<uint8_t *>(p);
  }

  const size_t bytes = n_layers * c->layer_elems() * c->elem;
  int rc = LTKV_OK;
  hipError_t e;
  if (bytes > 0) {
    if ((e = hipMalloc(&c->k, bytes)) != hipSuccess) rc = hip_fail(e, "hipMalloc(K pool)");
    else if ((e = hipMalloc(&c->v, bytes)) != hipSuccess) rc = hip_fail(e, "hipMalloc(V pool)");
    // zero cells; q8_0 quants are stored offset by 128, so a zero quant is 0x80
    else if ((e = hipMemset(c->k, c->q8() ? 0x80 : 0, bytes)) != hipSuccess) rc = hip_fail(e, "hipMemset(K pool)");
    else if ((e = hipMemset(c->v, c->q8() ? 0x80 : 0, bytes)) != hipSuccess) rc = hip_fail(e, "hipMemset(V pool)");
  }
  if (rc == LTKV_OK) {
    if ((e = hipMalloc((void **)&c->d_status, 4 * sizeof(int32_t))) != hipSuccess) rc = hip_fail(e, "hipMalloc(status)");
    else if ((e = hipMemset(c->d_status, 0, 4 * sizeof(int32_t))) != hipSuccess) rc = hip_fail(e, "hipMemset(status)");
  }
  const size_t sbytes = c->q8() ? n_layers * c->layer_scales() * 2 : 0;
  if (rc == LTKV_OK && sbytes > 0) {
    if ((e = hipMalloc(&c->ks, sbytes)) != hipSuccess) rc = hip_fail(e, "hipMalloc(K scales)");
    else if ((e = hipMalloc(&c->vs, sbytes)) != hipSuccess) rc = hip_fail(e, "hipMalloc(V scales)");
    else if ((e = hipMemset(c->ks, 0, sbytes)) != hipSuccess) rc = hip_fail(e, "hipMemset(K scales)");
    else if ((e = hipMemset(c->vs, 0, sbytes)) != hipSuccess) rc = hip_fail(e, "hipMemset(V scales)");
  }
  if (rc == LTKV_OK && (e = hipEventCreateWithFlags(&c->pairs_done, hipEventDisableTiming)) != hipSuccess)
    rc = hip_fail(e, "hipEventCreate");
  if (rc == LTKV_OK && (e = hipEventCreateWithFlags(&c->rt_done, hipEventDisableTiming)) != hipSuccess)
    rc = hip_fail(e, "hipEventCreate");
  if (rc != LTKV_OK) {
    ltkv_destroy(c);
    return rc;
  }
  *out = c;
  return LTKV_OK;
}

void ltkv_destroy(ltkv_cache *c) {
  if (!c) return;
  if (c->device != LTKV_NO_DEVICE) {
    DeviceGuard dg(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    else (void)hipDeviceSynchronize();
    if (c->pairs_done) (void)hipEventDestroy(c->pairs_done);
    if (c->h_pairs) (void)hipHostFree(c->h_pairs);
    if (c->d_pairs) (void)hipFree(c->d_pairs);
    if (c->d_order_counts) (void)hipFree(c->d_order_counts);
    if (c->d_order_pairs) (void)hipFree(c->d_order_pairs);
    if (c->ws) (void)hipFree(c->ws);
    if (c->d_status) (void)hipFree(c->d_status);
    if (c->rope) (void)hipFree(c->rope);
    if (c->plan.done) (void)hipEventDestroy(c->plan.done);
    if (c->plan.h) (void)hipHostFree(c->plan.h);
    if (c->plan.d) (void)hipFree(c->plan.d);
    if (c->k) (void)hipFree(c->k);
    if (c->v) (void)hipFree(c->v);
    if (c->ks) (void)hipFree(c->ks);
    if (c->vs) (void)hipFree(c->vs);
    if (c->rt_done) (void)hipEventDestroy(c->rt_done);
    if (c->h_rt_upd) (void)hipHostFree(c->h_rt_upd);
    if (c->d_rt_upd) (void)hipFree(c->d_rt_upd);
    if (c->d_rt) (void)hipFree(c->d_rt);
    if (c->d_rt_nb) (void)hipFree(c->d_rt_nb);
  }
  delete c;
}

int ltkv_set_stream(ltkv_cache *c, void *hip_stream) {
  if (!c) return fail(LTKV_ERR_ARG, "cache is null");
  c->stream = (hipStream_t)hip_stream;
  return LTKV_OK;
}

size_t ltkv_capacity(const ltkv_cache *c) { return c ? c->n_blocks * LTKV_BLOCK : 0; }
size_t ltkv_bytes(const ltkv_cache *c) {
  if (!c) return 0;
  return 2 * c->n_layers * (c->layer_elems() * c->elem + (c->q8() ? c->layer_scales() * 2 : 0));
}
size_t ltkv_len(const ltkv_cache *c, uint32_t seq) {
  if (!c) return 0;
  auto it = c->seqs.find(seq);
  return it == c->seqs.end() ? 0 : it->second.len;
}
size_t ltkv_free_blocks(const ltkv_cache *c) { return c ? c->free.size() : 0; }
size_t ltkv_n_blocks(const ltkv_cache *c) { return c ? c->n_blocks : 0; }
size_t ltkv_kv_dim(const ltkv_cache *c) { return c ? c->kv_dim : 0; }
uint32_t ltkv_refcount(const ltkv_cache *c, uint32_t block) {
  return (c && block < c->n_blocks) ? c->refs[block] : 0;
}
uint64_t ltkv_cow_copies(const ltkv_cache *c) { return c ? c->cow_copies : 0; }

int ltkv_append(ltkv_cache *c, uint32_t seq, size_t pos, uint32_t *block, uint32_t *slot) {
  if (!c || !block || !slot) return fail(LTKV_ERR_ARG, "null argument");
  const int rc = c->append_meta(seq, pos, block, slot);
  const int frc = c->flush_pending();
  return rc != LTKV_OK ? rc : frc;
}

int ltkv_append_batch(ltkv_cache *c, size_t n, const uint32_t *seqs, const uint64_t *pos,
                      int32_t *slot_mapping, size_t *n_done) {
  if (n_done) *n_done = 0;
  if (!c || (n && (!seqs || !pos || !slot_mapping))) return fail(LTKV_ERR_ARG, "null argument");
  int rc = LTKV_OK;
  size_t i = 0;
  for (; i < n; ++i) {
    uint32_t b, s;
    rc = c->append_meta(seqs[i], (size_t)pos[i], &b, &s);
    if (rc != LTKV_OK) break;
    slot_mapping[i] = (int32_t)(b * LTKV_BLOCK + s);
  }
  if (n_done) *n_done = i;
  if (rc != LTKV_OK) {  // the claim's error wins over a copy launch failure
    char err[sizeof g_err];
    std::memcpy(err, g_err, sizeof err);
    (void)c->flush_pending();
    std::memcpy(g_err, err, sizeof err);
    return rc;
  }
  return c->flush_pending();
}

void ltkv_truncate(ltkv_cache *c, uint32_t seq, size_t from) {
  if (c) c->truncate(seq, from);
}

void ltkv_share(ltkv_cache *c, uint32_t src, uint32_t dst, size_t len) {
  if (c) c->share(src, dst, len);
}

int ltkv_block_table(const ltkv_cache *c, uint32_t seq, int32_t *out, size_t cap, size_t *n_blocks) {
  if (!c) return fail(LTKV_ERR_ARG, "cache is null");
  auto it = c->seqs.find(seq);
  const size_t nb = it == c->seqs.end() ? 0 : it->second.blocks.size();
  if (n_blocks) *n_blocks = nb;
  if (nb > cap) return fail(LTKV_ERR_RANGE, "table of seq %u has %zu blocks, capacity %zu", seq, nb, cap);
  if (nb && !out) return fail(LTKV_ERR_ARG, "out is null");
  if (nb) std::memcpy(out, it->second.blocks.data(), nb * sizeof(int32_t));
  return LTKV_OK;
}

int ltkv_block_tables(const ltkv_cache *c, size_t n, const uint32_t *seqs, int32_t *out,
                      size_t stride) {
  if (!c || (n && (!seqs || !out))) return fail(LTKV_ERR_ARG, "null argument");
  for (size_t i = 0; i < n; ++i) {
    auto it = c->seqs.find(seqs[i]);
    const size_t nb = it == c->seqs.end() ? 0 : it->second.blocks.size();
    if (nb > stride)
      return fail(LTKV_ERR_RANGE, "table of seq %u has %zu blocks, stride %zu", seqs[i], nb, stride);
    int32_t *row = out + i * stride;
    if (nb) std::memcpy(row, it->second.blocks.data(), nb * sizeof(int32_t));
    std::fill(row + nb, row + stride, -1);
  }
  return LTKV_OK;
}

int ltkv_init_free_order(ltkv_cache *c, const uint32_t *order, size_t n) {
  if (!c || (n && !order)) return fail(LTKV_ERR_ARG, "null argument");
  if (!c->seqs.empty() || c->free.size() != c->n_blocks)
    return fail(LTKV_ERR_ARG, "init_free_order needs a cache with no sequences");
  ++c->gen;
  if (n != c->n_blocks) return fail(LTKV_ERR_ARG, "order has %zu entries, cache has %zu blocks", n, c->n_blocks);
  std::vector<uint8_t> seen(n, 0);
  for (size_t i = 0; i < n; ++i) {
    if (order[i] >= n || seen[order[i]]) return fail(LTKV_ERR_ARG, "order is not a permutation");
    seen[order[i]] = 1;
  }
  c->free.clear();
  for (size_t i = n; i-- > 0;) c->free.push_back((int32_t)order[i]);
  return LTKV_OK;
}

namespace {

// Kernel 1 over n launch rows: source row i, or order[i] of n_rows with an order.
int write_rows(ltkv_cache *c, size_t layer, size_t n, const int32_t *d_slot_mapping, const float *d_k,
               const float *d_v, size_t src_stride, const int32_t *d_order, size_t n_rows) {
  if (!c) return fail(LTKV_ERR_ARG, "cache is null");
  if (c->device == LTKV_NO_DEVICE) return no_device();
  if (layer >= c->n_layers) return fail(LTKV_ERR_RANGE, "layer %zu out of range (%zu)", layer, c->n_layers);
  if (n == 0) return LTKV_OK;
  if (!d_slot_mapping || !d_k || !d_v) return fail(LTKV_ERR_ARG, "null device pointer");
  if (n_rows > (size_t)INT32_MAX) return fail(LTKV_ERR_ARG, "%zu rows exceed 2^31 - 1", n_rows);
  if (src_stride < c->kv_dim) return fail(LTKV_ERR_ARG, "src_stride must be >= kv_dim");
  if (c->kv_dim % 8 == 0) {  // 16-byte row pieces (other row lengths move element-wise)
    if (src_stride % 4 != 0) return fail(LTKV_ERR_ARG, "src_stride must be a multiple of 4");
    if (((uintptr_t)d_k | (uintptr_t)d_v) % 16 != 0)
      return fail(LTKV_ERR_ARG, "K/V rows must be 16-byte aligned");
  } else if (((uintptr_t)d_k | (uintptr_t)d_v) % 4 != 0) {
    return fail(LTKV_ERR_ARG, "K/V must be 4-byte aligned");
  }
  if ((uint64_t)n * c->kv_dim >= (1ull << 40)) return fail(LTKV_ERR_ARG, "too many rows for one launch");
  DeviceGuard dg(c->device);
  if (!dg.ok) return fail(LTKV_ERR_HIP, "hipSetDevice(%d) failed", c->device);
  if (c->q8())
    HIP_TRY(ltkv::launch_write_q8(c->geom, c->k_layer(layer), c->v_layer(layer), c->k_scales(layer),
                                  c->v_scales(layer), d_slot_mapping, d_k, d_v, (int64_t)n,
                                  (int64_t)src_stride, c->stream, d_order, (int64_t)n_rows),
            "write launch");
  else
    HIP_TRY(ltkv::launch_write(c->geom, c->k_layer(layer), c->v_layer(layer), d_slot_mapping, d_k,
                               d_v, (int64_t)n, (int64_t)src_stride, c->stream, d_order, (int64_t)n_rows),
            "write launch");
  return LTKV_OK;
}

}  // namespace

int ltkv_write(ltkv_cache *c, size_t layer, size_t n, const int32_t *d_slot_mapping,
               const float *d_k, const float *d_v, size_t src_stride) {
  return write_rows(c, layer, n, d_slot_mapping, d_k, d_v, src_stride, nullptr, n);
}

int ltkv_write_ordered(ltkv_cache *c, size_t layer, size_t n, const int32_t *d_slot_mapping,
                       const float *d_k, const float *d_v, size_t src_stride, size_t m,
                       const int32_t *d_order) {
  if (m > 0 && !d_order) return fail(LTKV_ERR_ARG, "null device pointer");
  return write_rows(c, layer, m, d_slot_mapping, d_k, d_v, src_stride, d_order, n);
}

int ltkv_cell_order(const ltkv_cache *c, size_t n, const int32_t *slot_mapping, int32_t *order,
                    size_t *m) {
  if (!c || !m) return fail(LTKV_ERR_ARG, "null argument");
  *m = 0;
  if (n == 0) return LTKV_OK;
  if (!slot_mapping || !order) return fail(LTKV_ERR_ARG, "null host pointer");
  if (n > (size_t)INT32_MAX) return fail(LTKV_ERR_ARG, "%zu rows exceed 2^31 - 1", n);
  const int64_t n_cells = (int64_t)c->n_blocks * LTKV_BLOCK;
  size_t k = 0;
  if ((uint64_t)c->n_blocks > 4 * (uint64_t)n) {
    // few rows against the pool: sort (cell, row) pairs
    std::vector<std::pair<int32_t, int32_t>> v;
    v.reserve(n);
    for (size_t i = 0; i < n; ++i)
      if (slot_mapping[i] >= 0 && slot_mapping[i] < n_cells) v.emplace_back(slot_mapping[i], (int32_t)i);
    std::sort(v.begin(), v.end());
    for (const auto &e : v) order[k++] = e.second;
  } else {
    // counting sort by block, stable: a block's rows in a batch are one
    // sequence's positions in increasing order (kv.rs:85-121 claims them so),
    // hence in increasing slot order
    std::vector<int32_t> start(c->n_blocks + 1, 0);
    for (size_t i = 0; i < n; ++i)
      if (slot_mapping[i] >= 0 && slot_mapping[i] < n_cells) ++start[(slot_mapping[i] >> 4) + 1];
    for (size_t b = 0; b < c->n_blocks; ++b) start[b + 1] += start[b];
    k = (size_t)start[c->n_blocks];
    for (size_t i = 0; i < n; ++i)
      if (slot_mapping[i] >= 0 && slot_mapping[i] < n_cells) order[start[slot_mapping[i] >> 4]++] = (int32_t)i;
  }
  *m = k;
  return LTKV_OK;
}

int ltkv_rope_init(ltkv_cache *c, float base, size_t rope_dim, size_t head_dim, int neox,
                   size_t max_positions) {
  if (!c) return fail(LTKV_ERR_ARG, "cache is null");
  if (c->device == LTKV_NO_DEVICE) return no_device();
  if (head_dim == 0 || head_dim % 8 != 0 || c->kv_dim % head_dim != 0)
    return fail(LTKV_ERR_ARG, "head_dim %zu must be a multiple of 8 dividing kv_dim %zu", head_dim, c->kv_dim);
  if (rope_dim == 0 || rope_dim % 8 != 0 || rope_dim > head_dim)
    return fail(LTKV_ERR_ARG, "rope_dim %zu must be a multiple of 8 and at most head_dim", rope_dim);
  if (max_positions == 0 || max_positions > (size_t)INT32_MAX / 2)
    return fail(LTKV_ERR_ARG, "max_positions out of range");
  if (!(base > 0.f)) return fail(LTKV_ERR_ARG, "rope base must be positive");
  // model.rs:263-265 (inv_freq) and 296-297 (angle, sin_cos), with the same
  // libm the reference calls (powf, sinf, cosf).
  const size_t half = rope_dim / 2;
  std::vector<float> inv(half);
  for (size_t i = 0; i < half; ++i) inv[i] = powf(base, -2.0f * (float)i / (float)rope_dim);
  std::vector<float> tab(max_positions * half * 2);
  for (size_t p = 0; p < max_positions; ++p)
    for (size_t i = 0; i < half; ++i) {
      const float a = (float)p * inv[i];
      tab[(p * half + i) * 2] = cosf(a);
      tab[(p * half + i) * 2 + 1] = sinf(a);
    }
  DeviceGuard dg(c->device);
  if (!dg.ok) return fail(LTKV_ERR_HIP, "hipSetDevice(%d) failed", c->device);
  if (c->rope) {  // enqueued appends may still read the old table
    HIP_TRY(c->stream ? hipStreamSynchronize(c->stream) : hipDeviceSynchronize(), "synchronize");
    HIP_TRY(hipFree(c->rope), "hipFree(rope table)");
    c->rope = nullptr;
  }
  HIP_TRY(hipMalloc((void **)&c->rope, tab.size() * sizeof(float)), "hipMalloc(rope table)");
  HIP_TRY(hipMemcpy(c->rope, tab.data(), tab.size() * sizeof(float), hipMemcpyHostToDevice),
          "hipMemcpy(rope table)");
  c->rope_geom.table = c->rope;
  c->rope_geom.max_pos = (int)max_positions;
  c->rope_geom.rope_dim = (int)rope_dim;
  c->rope_geom.head_dim = (int)head_dim;
  c->rope_geom.neox = neox ? 1 : 0;
  return LTKV_OK;
}

int ltkv_write_rope(ltkv_cache *c, size_t layer, size_t n, const int32_t *d_slot_mapping,
                    const int32_t *d_positions, const float *d_k, const float *d_v, size_t src_stride,
                    float *d_q, size_t q_stride, size_t n_heads) {
  if (!c) return fail(LTKV_ERR_ARG, "cache is null");
  if (c->device == LTKV_NO_DEVICE) return no_device();
  if (!c->rope) return fail(LTKV_ERR_ARG, "no RoPE table (ltkv_rope_init)");
  if (layer >= c->n_layers) return fail(LTKV_ERR_RANGE, "layer %zu out of range (%zu)", layer, c->n_layers);
  if (n == 0) return LTKV_OK;
  if (!d_slot_mapping || !d_positions || !d_k || !d_v) return fail(LTKV_ERR_ARG, "null device pointer");
  if (src_stride < c->kv_dim || src_stride % 4 != 0)
    return fail(LTKV_ERR_ARG, "src_stride must be >= kv_dim and a multiple of 4");
  const size_t hd = (size_t)c->rope_geom.head_dim;
  if (c->q8() && hd % 32 != 0)
    return fail(LTKV_ERR_ARG, "the Q8_0 RoPE append needs head_dim a multiple of 32 (whole scale groups per head)");
  if (d_q && (n_heads == 0 || q_stride < n_heads * hd || q_stride % 4 != 0))
    return fail(LTKV_ERR_ARG, "q_stride must be >= n_heads * head_dim and a multiple of 4");
  if (((uintptr_t)d_k | (uintptr_t)d_v | (uintptr_t)d_q) % 16 != 0)
    return fail(LTKV_ERR_ARG, "K/V/Q rows must be 16-byte aligned");
  const uint64_t per = c->kv_dim / 8 * 2 + (d_q ? n_heads * hd / 8 : 0);
  if ((uint64_t)n * per >= (1ull << 32) - 256) return fail(LTKV_ERR_ARG, "too many rows for one launch");
  DeviceGuard dg(c->device);
  if (!dg.ok) return fail(LTKV_ERR_HIP, "hipSetDevice(%d) failed", c->device);
  if (c->q8())
    HIP_TRY(ltkv::launch_write_rope_q8(c->geom, c->k_layer(layer), c->v_layer(layer), c->k_scales(layer),
                                       c->v_scales(layer), d_slot_mapping, d_positions, d_k, d_v, d_q,
                                       (int64_t)n, (int64_t)src_stride, (int64_t)q_stride, (int)n_heads,
                                       c->rope_geom, c->stream),
            "write_rope launch");
  else
    HIP_TRY(ltkv::launch_write_rope(c->geom, c->k_layer(layer), c->v_layer(layer), d_slot_mapping,
                                    d_positions, d_k, d_v, d_q, (int64_t)n, (int64_t)src_stride,
                                    (int64_t)q_stride, (int)n_heads, c->rope_geom, c->stream),
            "write_rope launch");
  return LTKV_OK;
}

int ltkv_copy_blocks(ltkv_cache *c, size_t n, const int32_t *d_pairs) {
  if (!c) return fail(LTKV_ERR_ARG, "cache is null");
  if (c->device == LTKV_NO_DEVICE) return no_device();
  if (n == 0) return LTKV_OK;
  if (!d_pairs) return fail(LTKV_ERR_ARG, "null device pointer");
  DeviceGuard dg(c->device);
  if (!dg.ok) return fail(LTKV_ERR_HIP, "hipSetDevice(%d) failed", c->device);
  if (n > (size_t)INT32_MAX) return fail(LTKV_ERR_ARG, "%zu copy pairs exceed 2^31 - 1", n);
  const int64_t max_pairs = ltkv::copy_max_pairs(c->geom, (int)c->n_layers, n >= kCopyOrderMinPairs);
  if ((int64_t)n > max_pairs)
    return fail(LTKV_ERR_ARG, "%zu copy pairs exceed the %lld one launch takes at this pool shape", n,
                (long long)max_pairs);
  const int32_t *pairs = d_pairs;
  if (n >= kCopyOrderMinPairs) {
    // Large batch: bucket the pairs by destination first (three small
    // launches), so the copy writes in ascending destination order.
    const size_t buckets = (size_t)ltkv::copy_order_buckets((int64_t)c->n_blocks);
    if (n > c->order_cap) {
      if (c->d_order_pairs) {
        // the old buffer may still be read by an enqueued copy
        HIP_TRY(c->stream ? hipStreamSynchronize(c->stream) : hipDeviceSynchronize(), "synchronize");
        (void)hipFree(c->d_order_pairs);
      }
      c->d_order_pairs = nullptr;
      c->order_cap = 0;
      HIP_TRY(hipMalloc((void **)&c->d_order_pairs, n * 2 * sizeof(int32_t)), "hipMalloc(copy order)");
      c->order_cap = n;
    }
    if (!c->d_order_counts) {
      HIP_TRY(hipMalloc((void **)&c->d_order_counts, buckets * 2 * sizeof(int32_t)), "hipMalloc(copy order)");
      if (hipMemset(c->d_order_counts, 0, buckets * 2 * sizeof(int32_t)) != hipSuccess) {
        (void)hipFree(c->d_order_counts);
        c->d_order_counts = nullptr;
        return fail(LTKV_ERR_HIP, "hipMemset(copy order) failed");
      }
    }
    const hipError_t e = ltkv::launch_copy_order(d_pairs, (int64_t)n, (int64_t)c->n_blocks, c->d_order_counts,
                                                 c->d_order_counts + buckets, c->d_order_pairs, c->stream);
    if (e != hipSuccess) {
      // The counts may be left non-zero: start from fresh ones next time
      // (once whatever was enqueued has finished with them).
      (void)(c->stream ? hipStreamSynchronize(c->stream) : hipDeviceSynchronize());
      (void)hipFree(c->d_order_counts);
      c->d_order_counts = nullptr;
      return fail(LTKV_ERR_HIP, "copy order launch: %s", hipGetErrorString(e));
    }
    pairs = c->d_order_pairs;
  }
  const bool bulk = n >= kCopyOrderMinPairs;
  HIP_TRY(ltkv::launch_copy_blocks(c->geom, (int)c->n_layers, c->k, c->v, pairs, (int64_t)n, bulk, c->stream),
          "copy_blocks launch");
  if (c->q8())
    HIP_TRY(ltkv::launch_copy_blocks(c->sgeom, (int)c->n_layers, c->ks, c->vs, pairs, (int64_t)n, bulk,
                                     c->stream),
            "copy_blocks launch (scales)");
  return LTKV_OK;
}

int ltkv_gather(ltkv_cache *c, size_t layer, size_t n, const int32_t *d_tables,
                size_t table_stride, const int32_t *d_lens, const int64_t *d_out_offsets,
                void *d_k_out, void *d_v_out) {
  if (!c) return fail(LTKV_ERR_ARG, "cache is null");
  if (c->device == LTKV_NO_DEVICE) return no_device();
  if (layer >= c->n_layers) return fail(LTKV_ERR_RANGE, "layer %zu out of range (%zu)", layer, c->n_layers);
  if (c->q8()) return fail(LTKV_ERR_ARG, "gather has no Q8_0 form");
  if (n == 0 || table_stride == 0) return LTKV_OK;
  if (!d_tables || !d_lens || !d_out_offsets || !d_k_out || !d_v_out)
    return fail(LTKV_ERR_ARG, "null device pointer");
  if (((uintptr_t)d_k_out | (uintptr_t)d_v_out) % 16 != 0)
    return fail(LTKV_ERR_ARG, "outputs must be 16-byte aligned");
  // One work-group of 1024 threads per 16 KiB of a block's K or V.
  const uint64_t row_bytes = (uint64_t)c->kv_dim * c->geom.elem;
  const uint64_t chunks = (row_bytes + 1023) / 1024;
  if ((uint64_t)n * table_stride * 2 * chunks * 1024 >= (1ull << 32))
    return fail(LTKV_ERR_ARG, "n * table_stride too large for one launch");
  DeviceGuard dg(c->device);
  if (!dg.ok) return fail(LTKV_ERR_HIP, "hipSetDevice(%d) failed", c->device);
  HIP_TRY(ltkv::launch_gather(c->geom, c->k_layer(layer), c->v_layer(layer), d_tables,
                              (int64_t)table_stride, d_lens, d_out_offsets, (int64_t)n, d_k_out,
                              d_v_out, c->d_status, c->stream),
          "gather launch");
  return LTKV_OK;
}

int ltkv_set_attention_engine(ltkv_cache *c, int engine) {
  if (!c) return fail(LTKV_ERR_ARG, "cache is null");
  if (engine != LTKV_ENGINE_AUTO && engine != LTKV_ENGINE_VALU)
    return fail(LTKV_ERR_ARG, "unknown attention engine %d", engine);
  if (engine == LTKV_ENGINE_VALU && c->elem == 1)
    return fail(LTKV_ERR_ARG, "the vector-ALU engine serves f16 and f32 pools, not Q8_0");
  c->attn_engine = engine;
  return LTKV_OK;
}

int ltkv_set_attention_partition(ltkv_cache *c, size_t tokens) {
  if (!c) return fail(LTKV_ERR_ARG, "cache is null");
  if (tokens % 64 != 0 || tokens > (size_t{1} << 30))
    return fail(LTKV_ERR_ARG, "partition must be a multiple of 64 tokens, at most 2^30");
  c->attn_part_tokens = tokens;
  return LTKV_OK;
}

namespace {

// Decode attention over explicit tables (rows == nullptr: query i reads row
// i) or over the resident tables (query i reads row rows[i]); lengths are cut
// to max_len tokens, which sizes the grid.
// The partials go to the cache's workspace (grown on demand), or with
// use_scratch to the device's static scratch, which is never grown: a launch
// that needs more fails with LTKV_ERR_ARG and nothing is allocated.
int decode_attention(ltkv_cache *c, size_t layer, size_t n, size_t n_heads, size_t head_dim,
                     float scale, const float *d_q, const int32_t *d_tables, size_t table_stride,
                     const int32_t *d_rows, size_t n_rows, size_t max_len, const int32_t *d_lens,
                     float *d_out, size_t group, const int32_t *d_new_slots = nullptr,
                     const float *d_new_k = nullptr, const float *d_new_v = nullptr,
                     size_t new_stride = 0, bool use_scratch = false) {
  // A query's partition size depends on its own length only (or is fixed by
  // ltkv_set_attention_partition), so its result is bit-identical whatever
  // else is in the batch (the reference's property, engine/README.md:102).
  // max_len only bounds the grid.
  int part = (int)c->attn_part_tokens;  // 0: the shape's per-query policy
  const bool valu = c->attn_engine == LTKV_ENGINE_VALU && c->elem == 2;
  if (part == 0) part = ltkv::attention_part_policy((int)c->elem, (int)group, (int)(c->kv_dim / head_dim), valu);
  const int parts = ltkv::max_partitions((int64_t)max_len, part);
  const int split = ltkv::attention_split((int)c->elem, (int)group, (int)(c->kv_dim / head_dim));
  const size_t max_parts = (size_t)parts * split;
  if ((uint64_t)n * (n_heads / group) * max_parts * 256 >= (1ull << 32))
    return fail(LTKV_ERR_ARG, "attention grid too large for one launch");
  // Shapes outside the tuned kernels run the generic kernel over whole
  // contexts: no partition partials, so no workspace.
  const bool tuned = ltkv::attention_tuned((int)c->elem, (int)head_dim, (int)group);
  const ltkv::AttnWorkspace ws =
      tuned ? ltkv::attention_workspace((int64_t)n, (int)n_heads, (int)head_dim, (int)max_parts)
            : ltkv::AttnWorkspace{0, 0, 0};
  uint8_t *base = nullptr;
  if (use_scratch) {
    if ((size_t)ws.bytes > ltkv::kScratchBytes)
      return fail(LTKV_ERR_ARG,
                  "attention needs %lld bytes of partition partials, more than the %zu bytes of the "
                  "no-allocation scratch",
                  (long long)ws.bytes, ltkv::kScratchBytes);
    base = c->scratch;
  } else {
    if (int rc = ensure_workspace(c, (size_t)ws.bytes)) return rc;
    base = c->ws;
  }
  ltkv::AttnArgs a = attn_args(c, layer, n, n_heads, head_dim, scale, d_q, d_out, ws, part,
                               (int)max_parts, base);
  a.split = split;
  a.tables = d_tables;
  a.table_stride = (int64_t)table_stride;
  a.rows = d_rows;
  a.n_rows = (int64_t)n_rows;
  a.max_len = (int64_t)max_len;
  a.lens = d_lens;
  a.new_slots = d_new_slots;
  a.new_k = d_new_k;
  a.new_v = d_new_v;
  a.new_stride = (int64_t)new_stride;
  HIP_TRY(ltkv::launch_decode_attention(head_geom(c, head_dim), a, c->stream),
          "decode attention launch");
  return LTKV_OK;
}

}  // namespace

int ltkv_decode_attention(ltkv_cache *c, size_t layer, size_t n, size_t n_heads, size_t head_dim,
                          float scale, const float *d_q, const int32_t *d_tables,
                          size_t table_stride, const int32_t *d_lens, float *d_out) {
  if (!c) return fail(LTKV_ERR_ARG, "cache is null");
  if (c->device == LTKV_NO_DEVICE) return no_device();
  if (layer >= c->n_layers) return fail(LTKV_ERR_RANGE, "layer %zu out of range (%zu)", layer, c->n_layers);
  size_t group = 0;
  if (int rc = check_attention_shape(c, n_heads, head_dim, &group)) return rc;
  if (n == 0) return LTKV_OK;
  if (table_stride == 0) return fail(LTKV_ERR_ARG, "table_stride must be > 0");
  if (!d_q || !d_tables || !d_lens || !d_out) return fail(LTKV_ERR_ARG, "null device pointer");
  if (((uintptr_t)d_q) % 16 != 0) return fail(LTKV_ERR_ARG, "q must be 16-byte aligned");
  DeviceGuard dg(c->device);
  if (!dg.ok) return fail(LTKV_ERR_HIP, "hipSetDevice(%d) failed", c->device);
  return decode_attention(c, layer, n, n_heads, head_dim, scale, d_q, d_tables, table_stride, nullptr,
                          0, table_stride * LTKV_BLOCK, d_lens, d_out, group);
}

int ltkv_decode_attention_noalloc(ltkv_cache *c, size_t layer, size_t n, size_t n_heads,
                                  size_t head_dim, float scale, const float *d_q,
                                  const int32_t *d_tables, size_t table_stride, const int32_t *d_lens,
                                  float *d_out) {
  if (!c) return fail(LTKV_ERR_ARG, "cache is null");
  if (c->device == LTKV_NO_DEVICE) return no_device();
  if (layer >= c->n_layers) return fail(LTKV_ERR_RANGE, "layer %zu out of range (%zu)", layer, c->n_layers);
  size_t group = 0;
  if (int rc = check_attention_shape(c, n_heads, head_dim, &group)) return rc;
  if (n == 0) return LTKV_OK;
  if (table_stride == 0) return fail(LTKV_ERR_ARG, "table_stride must be > 0");
  if (!d_q || !d_tables || !d_lens || !d_out) return fail(LTKV_ERR_ARG, "null device pointer");
  if (((uintptr_t)d_q) % 16 != 0) return fail(LTKV_ERR_ARG, "q must be 16-byte aligned");
  if (!c->scratch) return fail(LTKV_ERR_HIP, "no-allocation scratch unavailable on device %d", c->device);
  DeviceGuard dg(c->device);
  if (!dg.ok) return fail(LTKV_ERR_HIP, "hipSetDevice(%d) failed", c->device);
  return decode_attention(c, layer, n, n_heads, head_dim, scale, d_q, d_tables, table_stride, nullptr,
                          0, table_stride * LTKV_BLOCK, d_lens, d_out, group, nullptr, nullptr, nullptr, 0,
                          true);
}

int ltkv_append_decode_attention(ltkv_cache *c, size_t layer, size_t n, size_t n_heads,
                                 size_t head_dim, float scale, const float *d_q,
                                 const int32_t *d_tables, size_t table_stride, const int32_t *d_lens,
                                 const int32_t *d_slot_mapping, const float *d_k, const float *d_v,
                                 size_t src_stride, float *d_out) {
  if (!c) return fail(LTKV_ERR_ARG, "cache is null");
  if (c->device == LTKV_NO_DEVICE) return no_device();
  if (layer >= c->n_layers) return fail(LTKV_ERR_RANGE, "layer %zu out of range (%zu)", layer, c->n_layers);
  size_t group = 0;
  if (int rc = check_attention_shape(c, n_heads, head_dim, &group)) return rc;
  if (n == 0) return LTKV_OK;
  if (table_stride == 0) return fail(LTKV_ERR_ARG, "table_stride must be > 0");
  if (!d_q || !d_tables || !d_lens || !d_out || !d_slot_mapping || !d_k || !d_v)
    return fail(LTKV_ERR_ARG, "null device pointer");
  if (((uintptr_t)d_q) % 16 != 0) return fail(LTKV_ERR_ARG, "q must be 16-byte aligned");
  if (src_stride < c->kv_dim || src_stride % 4 != 0)
    return fail(LTKV_ERR_ARG, "src_stride must be >= kv_dim and a multiple of 4");
  if (((uintptr_t)d_k | (uintptr_t)d_v) % 16 != 0) return fail(LTKV_ERR_ARG, "K/V rows must be 16-byte aligned");
  if (c->elem != 2 || !ltkv::attention_tuned(2, (int)head_dim, (int)group) ||
      c->attn_engine == LTKV_ENGINE_VALU) {
    // fused only on f16 pools of the tuned shapes with the matrix-core kernel:
    // otherwise append, then attention, as two launches
    if (int rc = ltkv_write(c, layer, n, d_slot_mapping, d_k, d_v, src_stride)) return rc;
    return ltkv_decode_attention(c, layer, n, n_heads, head_dim, scale, d_q, d_tables, table_stride,
                                 d_lens, d_out);
  }
  DeviceGuard dg(c->device);
  if (!dg.ok) return fail(LTKV_ERR_HIP, "hipSetDevice(%d) failed", c->device);
  return decode_attention(c, layer, n, n_heads, head_dim, scale, d_q, d_tables, table_stride, nullptr,
                          0, table_stride * LTKV_BLOCK, d_lens, d_out, group, d_slot_mapping, d_k, d_v,
                          src_stride);
}

int ltkv_decode_attention_rows(ltkv_cache *c, size_t layer, size_t n, size_t n_heads,
                               size_t head_dim, float scale, const float *d_q, const int32_t *d_rows,
                               const int32_t *d_lens, float *d_out) {
  if (!c) return fail(LTKV_ERR_ARG, "cache is null");
  if (c->device == LTKV_NO_DEVICE) return no_device();
  if (layer >= c->n_layers) return fail(LTKV_ERR_RANGE, "layer %zu out of range (%zu)", layer, c->n_layers);
  size_t group = 0;
  if (int rc = check_attention_shape(c, n_heads, head_dim, &group)) return rc;
  if (n == 0) return LTKV_OK;
  if (!d_q || !d_rows || !d_lens || !d_out) return fail(LTKV_ERR_ARG, "null device pointer");
  if (((uintptr_t)d_q) % 16 != 0) return fail(LTKV_ERR_ARG, "q must be 16-byte aligned");
  DeviceGuard dg(c->device);
  if (!dg.ok) return fail(LTKV_ERR_HIP, "hipSetDevice(%d) failed", c->device);
  if (int rc = sync_tables(c)) return rc;
  // No query reads past the longest live table.
  const size_t max_len = std::max<size_t>(max_table_blocks(c), 1) * LTKV_BLOCK;
  return decode_attention(c, layer, n, n_heads, head_dim, scale, d_q, c->d_rt, c->rt_width, d_rows,
                          c->rt_rows, max_len, d_lens, d_out, group);
}

int ltkv_seq_rows(const ltkv_cache *c, size_t n, const uint32_t *seqs, int32_t *rows) {
  if (!c) return fail(LTKV_ERR_ARG, "cache is null");
  if (n > 0 && (!seqs || !rows)) return fail(LTKV_ERR_ARG, "null argument");
  for (size_t i = 0; i < n; ++i) {
    const auto it = c->rt_row.find(seqs[i]);
    rows[i] = it == c->rt_row.end() ? -1 : it->second;
  }
  return LTKV_OK;
}

int ltkv_sync_tables(ltkv_cache *c) {
  if (!c) return fail(LTKV_ERR_ARG, "cache is null");
  if (c->device == LTKV_NO_DEVICE) return no_device();
  DeviceGuard dg(c->device);
  if (!dg.ok) return fail(LTKV_ERR_HIP, "hipSetDevice(%d) failed", c->device);
  return sync_tables(c);
}

int ltkv_resident_tables(ltkv_cache *c, const int32_t **d_tables, const int32_t **d_lengths,
                         size_t *stride, size_t *n_rows) {
  if (!c) return fail(LTKV_ERR_ARG, "cache is null");
  if (c->device == LTKV_NO_DEVICE) return no_device();
  DeviceGuard dg(c->device);
  if (!dg.ok) return fail(LTKV_ERR_HIP, "hipSetDevice(%d) failed", c->device);
  if (int rc = sync_tables(c)) return rc;
  if (d_tables) *d_tables = c->d_rt;
  if (d_lengths) *d_lengths = c->d_rt_nb;
  if (stride) *stride = c->rt_width;
  if (n_rows) *n_rows = c->rt_rows;
  return LTKV_OK;
}

int ltkv_slot_mapping(ltkv_cache *c, size_t n, const int32_t *d_rows, const int64_t *d_pos,
                      int32_t *d_slot_mapping) {
  if (!c) return fail(LTKV_ERR_ARG, "cache is null");
  if (c->device == LTKV_NO_DEVICE) return no_device();
  if (n == 0) return LTKV_OK;
  if (!d_rows || !d_pos || !d_slot_mapping) return fail(LTKV_ERR_ARG, "null device pointer");
  DeviceGuard dg(c->device);
  if (!dg.ok) return fail(LTKV_ERR_HIP, "hipSetDevice(%d) failed", c->device);
  if (int rc = sync_tables(c)) return rc;
  HIP_TRY(ltkv::launch_slot_mapping(c->d_rt, c->d_rt_nb, (int64_t)c->rt_width, (int64_t)c->rt_rows,
                                    d_rows, d_pos, (int64_t)n, d_slot_mapping, c->stream),
          "slot mapping launch");
  return LTKV_OK;
}

int ltkv_read_resident_tables(ltkv_cache *c, int32_t *h_tables, int32_t *h_lengths) {
  if (!c || !h_tables || !h_lengths) return fail(LTKV_ERR_ARG, "null argument");
  if (c->device == LTKV_NO_DEVICE) return no_device();
  DeviceGuard dg(c->device);
  if (!dg.ok) return fail(LTKV_ERR_HIP, "hipSetDevice(%d) failed", c->device);
  if (int rc = sync_tables(c)) return rc;
  HIP_TRY(hipMemcpyAsync(h_tables, c->d_rt, c->rt_rows * c->rt_width * sizeof(int32_t),
                         hipMemcpyDeviceToHost, c->stream),
          "hipMemcpyAsync(resident tables)");
  HIP_TRY(hipMemcpyAsync(h_lengths, c->d_rt_nb, c->rt_rows * sizeof(int32_t), hipMemcpyDeviceToHost,
                         c->stream),
          "hipMemcpyAsync(resident table lengths)");
  HIP_TRY(c->stream ? hipStreamSynchronize(c->stream) : hipDeviceSynchronize(), "synchronize");
  return take_status(c);
}

int ltkv_table_uploads(const ltkv_cache *c, uint64_t *entries) {
  if (!c || !entries) return fail(LTKV_ERR_ARG, "null argument");
  *entries = c->rt_uploaded;
  return LTKV_OK;
}

int ltkv_plan_attention(ltkv_cache *c, size_t n, const uint32_t *seqs, const uint32_t *lens,
                        size_t n_heads, size_t head_dim, unsigned flags) {
  if (!c) return fail(LTKV_ERR_ARG, "cache is null");
  c->plan.valid = false;
  size_t group = 0;
  if (int rc = check_attention_shape(c, n_heads, head_dim, &group)) return rc;
  if (n && (!seqs || !lens)) return fail(LTKV_ERR_ARG, "null argument");
  if (n > (size_t)INT32_MAX / 64) return fail(LTKV_ERR_ARG, "batch of %zu queries is too large", n);
  if (flags & ~(unsigned)(LTKV_PLAN_SHARED_PREFIX | LTKV_PLAN_F16_PRODUCTS))
    return fail(LTKV_ERR_ARG, "unknown plan flags 0x%x", flags);
  if (int rc = build_plan(c, n, seqs, lens, n_heads, head_dim, group, flags)) return rc;
  c->plan.f16_products = (flags & LTKV_PLAN_F16_PRODUCTS) != 0;
  if (c->device != LTKV_NO_DEVICE) {
    if (int rc = upload_plan(c)) return rc;
  }
  c->plan.valid = true;
  c->plan.gen = c->gen;
  return LTKV_OK;
}

int ltkv_planned_attention(ltkv_cache *c, size_t layer, float scale, const float *d_q, float *d_out) {
  if (!c) return fail(LTKV_ERR_ARG, "cache is null");
  if (c->device == LTKV_NO_DEVICE) return no_device();
  const AttnPlan &P = c->plan;
  if (!P.valid) return fail(LTKV_ERR_ARG, "no attention plan (ltkv_plan_attention)");
  if (P.gen != c->gen)
    return fail(LTKV_ERR_ARG, "the attention plan is stale: block tables changed after ltkv_plan_attention");
  if (layer >= c->n_layers) return fail(LTKV_ERR_RANGE, "layer %zu out of range (%zu)", layer, c->n_layers);
  if (P.n == 0) return LTKV_OK;
  if (!d_q || !d_out) return fail(LTKV_ERR_ARG, "null device pointer");
  if (((uintptr_t)d_q) % 16 != 0) return fail(LTKV_ERR_ARG, "q must be 16-byte aligned");
  const size_t group = P.n_heads / (c->kv_dim / P.head_dim);
  const bool grouped = P.groups > 0;
  // Grouped plans are batch-dependent anyway: when every query's remainder is
  // short (forks reading a few private blocks), their per-query pass takes
  // the plan's partition unless one is fixed; long remainders keep the
  // per-query policy.
  // Such remainders are not cut further (the q8_0 decode cut): a remainder in
  // one partition lets its wave fold the group partials itself, with no merge
  // launch (q8_0 config-3 step: the merge took ~11 us of ~98).
  int part = (int)c->attn_part_tokens;
  const bool short_rem = grouped && part == 0 && P.sstride * LTKV_BLOCK <= kShortRemainder;
  if (short_rem) part = P.suffix_part;
  else if (part == 0)
    part = ltkv::attention_part_policy((int)c->elem, (int)group, (int)(c->kv_dim / P.head_dim),
                                       c->attn_engine == LTKV_ENGINE_VALU && c->elem == 2);
  const int parts = ltkv::max_partitions((int64_t)(P.sstride * LTKV_BLOCK), part);
  const int split =
      short_rem ? 1 : ltkv::attention_split((int)c->elem, (int)group, (int)(c->kv_dim / P.head_dim));
  const size_t max_parts = (size_t)parts * split;
  if ((uint64_t)P.n * (P.n_heads / group) * max_parts * 256 >= (1ull << 32))
    return fail(LTKV_ERR_ARG, "attention grid too large for one launch");

  DeviceGuard dg(c->device);
  if (!dg.ok) return fail(LTKV_ERR_HIP, "hipSetDevice(%d) failed", c->device);
  const ltkv::AttnWorkspace ws = ltkv::attention_workspace(
      (int64_t)P.n, (int)P.n_heads, (int)P.head_dim, (int)max_parts, grouped);
  const size_t pre_slots = grouped ? P.n * P.n_heads * (size_t)P.max_pre_parts : 0;
  const size_t pre_o_off = ((size_t)ws.bytes + 255) / 256 * 256;
  const size_t pre_ml_off = pre_o_off + pre_slots * P.head_dim * 4;
  if (int rc = ensure_workspace(c, pre_ml_off + pre_slots * 2 * 4)) return rc;
  const int32_t *d = reinterpret_cast<const int32_t *>(P.d);
  const ltkv::PoolGeom g = head_geom(c, P.head_dim);
  ltkv::AttnArgs a = attn_args(c, layer, P.n, P.n_heads, P.head_dim, scale, d_q, d_out, ws, part,
                               (int)max_parts, c->ws);
  a.split = split;
  // Short remainders in one partition each and no group-only queries: the
  // decode kernel writes every output itself (folding group partials).
  a.merge_free = grouped && part > 0 && P.max_suffix <= (size_t)(part / split) && !P.empty_with_groups;
  a.pass_empty = grouped && P.pass_empty;
  a.tables = d + P.off_stables;
  a.table_stride = (int64_t)P.sstride;
  a.max_len = (int64_t)(P.sstride * LTKV_BLOCK);
  a.lens = d + P.off_slens;
  if (P.n_pass < P.n) {  // only the queries that groups did not complete
    a.n = (int64_t)P.n_pass;
    a.qmap = d + P.off_qmap;
  }
  if (grouped) {
    a.pre_parts = d + P.off_pre;
    a.pre_o = (float *)(c->ws + pre_o_off);
    a.pre_ml = (float *)(c->ws + pre_ml_off);
    a.max_pre_parts = P.max_pre_parts;
    ltkv::MqArgs m{};
    m.k_layer = a.k_layer;
    m.v_layer = a.v_layer;
    m.k_scale = a.k_scale;
    m.v_scale = a.v_scale;
    m.q = d_q;
    m.tables = d + P.off_tables;
    m.jobs = reinterpret_cast<const ltkv::MqJob *>(d + P.off_jobs);
    m.n_jobs = P.n_jobs;
    m.members = d + P.off_members;
    m.pre_o = (float *)a.pre_o;
    m.pre_ml = (float *)a.pre_ml;
    m.out = d_out;
    m.n_heads = (int)P.n_heads;
    m.n_kv_heads = a.n_kv_heads;
    m.head_dim = (int)P.head_dim;
    m.scale = scale;
    m.max_pre_parts = P.max_pre_parts;
    m.f16_products = P.f16_products;
    // The two passes run one after the other: the shared-prefix kernel's
    // footprint (two waves per SIMD) leaves no room to overlap them.
    HIP_TRY(ltkv::launch_mq_attention(g, m, c->stream), "shared-prefix attention launch");
    if (P.groups_only) return LTKV_OK;  // the groups wrote every output
  }
  HIP_TRY(ltkv::launch_decode_attention(g, a, c->stream), "decode attention launch");
  return LTKV_OK;
}

int ltkv_plan_stats(const ltkv_cache *c, uint64_t out[6]) {
  if (!c || !out) return fail(LTKV_ERR_ARG, "null argument");
  const AttnPlan &P = c->plan;
  if (!P.valid) return fail(LTKV_ERR_ARG, "no attention plan (ltkv_plan_attention)");
  out[0] = P.n;
  out[1] = P.groups;
  out[2] = P.grouped;
  out[3] = P.shared_blocks;
  out[4] = (uint64_t)P.n_jobs;
  out[5] = P.stride;
  return LTKV_OK;
}

int ltkv_synchronize(ltkv_cache *c) {
  if (!c) return fail(LTKV_ERR_ARG, "cache is null");
  if (c->device == LTKV_NO_DEVICE) return no_device();
  DeviceGuard dg(c->device);
  if (!dg.ok) return fail(LTKV_ERR_HIP, "hipSetDevice(%d) failed", c->device);
  HIP_TRY(c->stream ? hipStreamSynchronize(c->stream) : hipDeviceSynchronize(), "synchronize");
  return take_status(c);
}

int ltkv_read_pool(ltkv_cache *c, size_t layer, void *h_k, void *h_v) {
  if (!c) return fail(LTKV_ERR_ARG, "cache is null");
  if (c->device == LTKV_NO_DEVICE) return no_device();
  if (layer >= c->n_layers) return fail(LTKV_ERR_RANGE, "layer %zu out of range (%zu)", layer, c->n_layers);
  if (!h_k || !h_v) return fail(LTKV_ERR_ARG, "null host pointer");
  DeviceGuard dg(c->device);
  if (!dg.ok) return fail(LTKV_ERR_HIP, "hipSetDevice(%d) failed", c->device);
  const size_t bytes = c->layer_elems() * c->elem;
  HIP_TRY(hipMemcpyAsync(h_k, c->k_layer(layer), bytes, hipMemcpyDeviceToHost, c->stream), "read K pool");
  HIP_TRY(hipMemcpyAsync(h_v, c->v_layer(layer), bytes, hipMemcpyDeviceToHost, c->stream), "read V pool");
  HIP_TRY(c->stream ? hipStreamSynchronize(c->stream) : hipDeviceSynchronize(), "synchronize");
  if (c->q8()) {  // stored bytes q + 128 back to int8 quants
    for (uint8_t *p : {static_cast<uint8_t *>(h_k), static_cast<uint8_t *>(h_v)})
      for (size_t i = 0; i < bytes; ++i) p[i] ^= 0x80;
  }
  return LTKV_OK;
}

int ltkv_read_scales(ltkv_cache *c, size_t layer, uint16_t *h_k, uint16_t *h_v) {
  if (!c) return fail(LTKV_ERR_ARG, "cache is null");
  if (c->device == LTKV_NO_DEVICE) return no_device();
  if (!c->q8()) return fail(LTKV_ERR_ARG, "only Q8_0 caches have scale pools");
  if (layer >= c->n_layers) return fail(LTKV_ERR_RANGE, "layer %zu out of range (%zu)", layer, c->n_layers);
  if (!h_k || !h_v) return fail(LTKV_ERR_ARG, "null host pointer");
  DeviceGuard dg(c->device);
  if (!dg.ok) return fail(LTKV_ERR_HIP, "hipSetDevice(%d) failed", c->device);
  const size_t bytes = c->layer_scales() * 2;
  HIP_TRY(hipMemcpyAsync(h_k, c->k_scales(layer), bytes, hipMemcpyDeviceToHost, c->stream), "read K scales");
  HIP_TRY(hipMemcpyAsync(h_v, c->v_scales(layer), bytes, hipMemcpyDeviceToHost, c->stream), "read V scales");
  HIP_TRY(c->stream ? hipStreamSynchronize(c->stream) : hipDeviceSynchronize(), "synchronize");
  return take_status(c);
}

int ltkv_rows(ltkv_cache *c, size_t layer, uint32_t seq, size_t n, void *h_k, void *h_v) {
  if (!c) return fail(LTKV_ERR_ARG, "cache is null");
  if (c->device == LTKV_NO_DEVICE) return no_device();
  if (c->q8()) return fail(LTKV_ERR_ARG, "rows has no Q8_0 form (ltkv_read_pool, ltkv_read_scales)");
  if (layer >= c->n_layers) return fail(LTKV_ERR_RANGE, "layer %zu out of range (%zu)", layer, c->n_layers);
  if (n == 0) return LTKV_OK;
  if (!h_k || !h_v) return fail(LTKV_ERR_ARG, "null host pointer");
  auto it = c->seqs.find(seq);
  const size_t nb = it == c->seqs.end() ? 0 : it->second.blocks.size();
  if ((n + LTKV_BLOCK - 1) / LTKV_BLOCK > nb)
    return fail(LTKV_ERR_RANGE, "rows(%u, %zu): sequence has %zu blocks", seq, n, nb);
  DeviceGuard dg(c->device);
  if (!dg.ok) return fail(LTKV_ERR_HIP, "hipSetDevice(%d) failed", c->device);
  // Staging: [table | len | offset] then K and V rows, in one device buffer.
  const size_t tb = (n + LTKV_BLOCK - 1) / LTKV_BLOCK;
  const size_t row_bytes = c->kv_dim * c->elem;
  const size_t off_pos = (tb * 4 + 4 + 7) / 8 * 8;  // int64 output offset, 8-aligned
  const size_t meta = (off_pos + 8 + 255) / 256 * 256;
  const size_t total = meta + 2 * n * row_bytes;
  uint8_t *d = nullptr;
  HIP_TRY(hipMalloc((void **)&d, total), "hipMalloc(rows staging)");
  std::vector<uint8_t> h(meta, 0);
  std::memcpy(h.data(), it->second.blocks.data(), tb * 4);
  const int32_t len = (int32_t)n;
  const int64_t off = 0;
  std::memcpy(h.data() + tb * 4, &len, 4);
  std::memcpy(h.data() + off_pos, &off, 8);
  hipError_t e = hipMemcpyAsync(d, h.data(), meta, hipMemcpyHostToDevice, c->stream);
  if (e == hipSuccess)
    e = ltkv::launch_gather(c->geom, c->k_layer(layer), c->v_layer(layer), (const int32_t *)d,
                            (int64_t)tb, (const int32_t *)(d + tb * 4), (const int64_t *)(d + off_pos),
                            1, d + meta, d + meta + n * row_bytes, c->d_status, c->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(h_k, d + meta, n * row_bytes, hipMemcpyDeviceToHost, c->stream);
  if (e == hipSuccess) e = hipMemcpyAsync(h_v, d + meta + n * row_bytes, n * row_bytes, hipMemcpyDeviceToHost, c->stream);
  {  // whatever was enqueued must be done with the staging before it is freed
    const hipError_t se = c->stream ? hipStreamSynchronize(c->stream) : hipDeviceSynchronize();
    if (e == hipSuccess) e = se;
  }
  (void)hipFree(d);
  if (e != hipSuccess) return hip_fail(e, "rows");
  return LTKV_OK;
}

int ltkv_write_row(ltkv_cache *c, size_t layer, uint32_t block, uint32_t slot, const float *h_k,
                   const float *h_v) {
  if (!c) return fail(LTKV_ERR_ARG, "cache is null");
  if (c->device == LTKV_NO_DEVICE) return no_device();
  if (layer >= c->n_layers) return fail(LTKV_ERR_RANGE, "layer %zu out of range (%zu)", layer, c->n_layers);
  if (block >= c->n_blocks || slot >= LTKV_BLOCK)
    return fail(LTKV_ERR_RANGE, "cell (%u, %u) out of range", block, slot);
  if (!h_k || !h_v) return fail(LTKV_ERR_ARG, "null host pointer");
  DeviceGuard dg(c->device);
  if (!dg.ok) return fail(LTKV_ERR_HIP, "hipSetDevice(%d) failed", c->device);
  // Staging: [slot mapping (16 bytes) | K row | V row].
  const size_t row = c->kv_dim * sizeof(float);
  const size_t total = 16 + 2 * row;
  std::vector<uint8_t> h(total, 0);
  const int32_t cell = (int32_t)(block * LTKV_BLOCK + slot);
  std::memcpy(h.data(), &cell, 4);
  std::memcpy(h.data() + 16, h_k, row);
  std::memcpy(h.data() + 16 + row, h_v, row);
  uint8_t *d = nullptr;
  HIP_TRY(hipMalloc((void **)&d, total), "hipMalloc(row staging)");
  hipError_t e = hipMemcpyAsync(d, h.data(), total, hipMemcpyHostToDevice, c->stream);
  if (e == hipSuccess && c->q8())
    e = ltkv::launch_write_q8(c->geom, c->k_layer(layer), c->v_layer(layer), c->k_scales(layer),
                              c->v_scales(layer), (const int32_t *)d, (const float *)(d + 16),
                              (const float *)(d + 16 + row), 1, (int64_t)c->kv_dim, c->stream);
  else if (e == hipSuccess)
    e = ltkv::launch_write(c->geom, c->k_layer(layer), c->v_layer(layer), (const int32_t *)d,
                           (const float *)(d + 16), (const float *)(d + 16 + row), 1,
                           (int64_t)c->kv_dim, c->stream);
  {  // whatever was enqueued must be done with the staging before it is freed
    const hipError_t se = c->stream ? hipStreamSynchronize(c->stream) : hipDeviceSynchronize();
    if (e == hipSuccess) e = se;
  }
  (void)hipFree(d);
  if (e != hipSuccess) return hip_fail(e, "write_row");
  return LTKV_OK;
}

}  // extern "C"
