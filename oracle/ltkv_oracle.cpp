// ltkv oracle: CPU restatement of the Langtrain engine's paged KV-cache path.
//
// TEST INFRASTRUCTURE ONLY. This file is the oracle that the HIP product is
// checked against, and the CPU baseline that bench.py times beside it. Only
// tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load the
// library built from it; the product (langtrain_studio_amd/) never does.
//
// What it restates (paths relative to the reference checkout):
//   * engine/crates/native/src/kv.rs:13-187   KvCache: 16-token blocks, LIFO free
//     stack, refcounts, append with copy-on-write, write (f32 -> f16 RNE),
//     rows, truncate, share, free_blocks.
//   * engine/crates/native/src/model.rs:158-172  dot(): 8 independent f32
//     partial sums, then a sequential tail, then sum(acc) + tail.
//   * engine/crates/native/src/model.rs:380-383,431-475  cell claim and the
//     attention closure: one task per (token, kv_head), K pass, per-head
//     softmax (max fold, expf, sequential sum, multiply by 1/sum), V pass.
//   * engine/crates/native/src/pool.rs:14,77-167,188-199  spin-then-park pool
//     that runs the attention tasks.
//
//   * engine/crates/native/src/quant.rs:785-791  quantize_block (int8 per 32
//     elements, scale amax / 127) and quant.rs:188-193 (Q8_0 block: f16 d
//     then 32 int8, read back as d * q) for the Q8_0 storage mode.
//
// Storage dtype: the reference stores f16 only (kv.rs:5-6,21-22). Mode F32
// is the same algorithm with the rounding step removed (no reference
// counterpart; used by the TinyLlama-shaped f32 workload). Mode Q8_0 stores
// each row as Q8_0 blocks (the KV cache type of the engine's llama.cpp
// backend, hardware.rs:173 / llama.rs:113-118); attention reads the
// dequantised rows d * q and is otherwise the same closure.
//
// Build: oracle/Makefile (g++ -O3 -ffp-contract=off; no FMA contraction,
// matching rustc's default).

#include <atomic>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <functional>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#if defined(__F16C__)
#include <immintrin.h>
#endif

namespace {

constexpr size_t kBlock = 16;  // kv.rs:13

// ---------------------------------------------------------------------------
// IEEE-754 binary16 conversions, written from the format definition.
// f32 -> f16 is round-to-nearest-even; NaN keeps the top 10 payload bits and
// is forced quiet (bit 9), which is what the `half` crate's from_f32 yields.
// ---------------------------------------------------------------------------
uint16_t f32_to_f16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t exp = (x >> 23) & 0xffu;
  const uint32_t man = x & 0x7fffffu;
  if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? (0x0200u | (man >> 13)) : 0u));
  const int e = (int)exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    // Result is subnormal (or zero): count units of 2^-24.
    const int shift = 14 - e;  // >= 14
    if (shift > 24) return (uint16_t)sign;
    const uint32_t m = man | 0x800000u;
    uint32_t q = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
  }
  uint32_t q = ((uint32_t)e << 10) | (man >> 13);
  const uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;  // carry may reach inf: correct
  return (uint16_t)(sign | q);
}

float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t bits;
  if (exp == 0x1fu) {
    bits = sign | 0x7f800000u | (man << 13);
  } else if (exp == 0) {
    if (man == 0) {
      bits = sign;
    } else {
      int e = -14;
      while (!(man & 0x400u)) { man <<= 1; --e; }
      man &= 0x3ffu;
      bits = sign | ((uint32_t)(e + 127) << 23) | (man << 13);
    }
  } else {
    bits = sign | ((exp - 15 + 127) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

// Row widening, as half's convert_to_f32_slice (model.rs:448,466).
void widen_row(const uint16_t *src, float *dst, size_t n) {
  size_t i = 0;
#if defined(__F16C__)
  for (; i + 8 <= n; i += 8)
    _mm256_storeu_ps(dst + i, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(src + i))));
#endif
  for (; i < n; ++i) dst[i] = f16_to_f32(src[i]);
}

// Row narrowing, as the per-element f16::from_f32 loop of kv.rs:125-130.
void narrow_row(const float *src, uint16_t *dst, size_t n) {
  size_t i = 0;
#if defined(__F16C__)
  for (; i + 8 <= n; i += 8)
    _mm_storeu_si128((__m128i *)(dst + i),
                     _mm256_cvtps_ph(_mm256_loadu_ps(src + i), _MM_FROUND_TO_NEAREST_INT));
#endif
  for (; i < n; ++i) dst[i] = f32_to_f16(src[i]);
}

// ---------------------------------------------------------------------------
// Spin-then-park pool (pool.rs:14-167). One job at a time; the caller works
// too; idle workers spin 500 us before parking with a 50 ms timed wait.
// ---------------------------------------------------------------------------
class Pool {
 public:
  explicit Pool(size_t threads) : threads_(threads ? threads : 1) {
    for (size_t i = 1; i < threads_; ++i) workers_.emplace_back([this] { worker(); });
  }
  ~Pool() {
    shutdown_.store(true, std::memory_order_release);
    {
      std::lock_guard<std::mutex> g(sleep_mu_);
      wake_.notify_all();
    }
    for (auto &t : workers_) t.join();
  }
  size_t threads() const { return threads_; }

  void run(size_t n, const std::function<void(size_t)> &f) {
    if (n == 0) return;
    if (n == 1 || threads_ == 1) {
      for (size_t i = 0; i < n; ++i) f(i);
      return;
    }
    std::lock_guard<std::mutex> gate(gate_);
    auto job = std::make_shared<Job>();
    job->f = &f;
    job->n = n;
    job->next.store(0);
    job->pending.store(n);
    {
      std::lock_guard<std::mutex> g(job_mu_);
      job_ = job;
    }
    generation_.fetch_add(1, std::memory_order_acq_rel);
    {
      std::lock_guard<std::mutex> g(sleep_mu_);
      if (sleeping_ > 0) wake_.notify_all();
    }
    work(*job);
    while (job->pending.load(std::memory_order_acquire) != 0) {
#if defined(__x86_64__)
      __builtin_ia32_pause();
#endif
    }
    std::lock_guard<std::mutex> g(job_mu_);
    job_.reset();
  }

 private:
  struct Job {
    const std::function<void(size_t)> *f = nullptr;
    size_t n = 0;
    std::atomic<size_t> next{0};
    std::atomic<size_t> pending{0};
  };

  static void work(Job &job) {
    for (;;) {
      const size_t i = job.next.fetch_add(1, std::memory_order_relaxed);
      if (i >= job.n) return;
      (*job.f)(i);
      job.pending.fetch_sub(1, std::memory_order_acq_rel);
    }
  }

  void worker() {
    size_t seen = generation_.load(std::memory_order_acquire);
    for (;;) {
      auto start = std::chrono::steady_clock::now();
      for (;;) {
        if (shutdown_.load(std::memory_order_acquire)) return;
        const size_t g = generation_.load(std::memory_order_acquire);
        if (g != seen) {
          seen = g;
          break;
        }
        if (std::chrono::steady_clock::now() - start > std::chrono::microseconds(500)) {
          std::unique_lock<std::mutex> lk(sleep_mu_);
          ++sleeping_;
          while (generation_.load(std::memory_order_acquire) == seen &&
                 !shutdown_.load(std::memory_order_acquire))
            wake_.wait_for(lk, std::chrono::milliseconds(50));
          --sleeping_;
          start = std::chrono::steady_clock::now();
          continue;
        }
#if defined(__x86_64__)
        __builtin_ia32_pause();
#endif
      }
      std::shared_ptr<Job> job;
      {
        std::lock_guard<std::mutex> g(job_mu_);
        job = job_;
      }
      if (job) work(*job);
    }
  }

  size_t threads_;
  std::vector<std::thread> workers_;
  std::atomic<size_t> generation_{0};
  std::mutex job_mu_;
  std::shared_ptr<Job> job_;
  std::mutex sleep_mu_;
  size_t sleeping_ = 0;
  std::condition_variable wake_;
  std::atomic<bool> shutdown_{false};
  std::mutex gate_;
};

// ---------------------------------------------------------------------------
// KvCache restatement (kv.rs:15-187).
// quant.rs:785-791: amax folded with f32::max (a NaN element is ignored),
// d = amax / 127, id = 1 / d (0 when d is 0), q = (v * id).round() as i8:
// round half away from zero, then Rust's saturating float -> int cast
// (NaN -> 0, beyond the range -> -128 / 127).
inline int8_t sat_i8(float r) {
  if (std::isnan(r)) return 0;
  if (r >= 127.0f) return 127;
  if (r <= -128.0f) return -128;
  return (int8_t)(int)r;
}
float quantize_block(const float *x, int8_t *q) {
  float amax = 0.0f;
  for (int i = 0; i < 32; ++i) amax = std::fmax(amax, std::fabs(x[i]));
  const float d = amax / 127.0f;
  const float id = d > 0.0f ? 1.0f / d : 0.0f;
  for (int i = 0; i < 32; ++i) q[i] = sat_i8(std::round(x[i] * id));
  return d;
}

// ---------------------------------------------------------------------------
struct Seq {
  std::vector<size_t> blocks;
  size_t len = 0;
};

struct OracleKv {
  size_t n_layers, kv_dim, n_blocks, elem;  // elem: 2 (f16), 4 (f32) or 1 (Q8_0 quants)
  std::vector<uint8_t> k, v;                 // [layer][block][slot][kv_dim]
  std::vector<uint16_t> ks, vs;              // Q8_0: f16 d per 32, [layer][block][slot][kv_dim/32]
  std::vector<uint32_t> refs;
  std::vector<size_t> free;  // stack; back() is popped first
  std::unordered_map<uint32_t, Seq> seqs;
  uint64_t cow_copies = 0;
  std::string err;

  OracleKv(size_t nl, size_t kvd, size_t n_tokens, size_t elem_bytes)
      : n_layers(nl), kv_dim(kvd), n_blocks((n_tokens + kBlock - 1) / kBlock), elem(elem_bytes) {
    const size_t size = n_layers * n_blocks * kBlock * kv_dim * elem;
    k.assign(size, 0);
    v.assign(size, 0);
    if (elem == 1) {
      ks.assign(size / 32, 0);
      vs.assign(size / 32, 0);
    }
    refs.assign(n_blocks, 0);
    free.reserve(n_blocks);
    for (size_t b = n_blocks; b-- > 0;) free.push_back(b);  // (0..n).rev(): pop gives 0,1,2..
  }

  size_t offset(size_t layer, size_t block, size_t slot) const {  // kv.rs:62-65
    return ((layer * n_blocks + block) * kBlock + slot) * kv_dim;
  }

  bool alloc(size_t *b) {  // kv.rs:67-74
    if (free.empty()) {
      err = "KV cache full";
      return false;
    }
    *b = free.back();
    free.pop_back();
    refs[*b] = 1;
    return true;
  }

  void release(size_t b) {  // kv.rs:76-81
    refs[b] -= 1;
    if (refs[b] == 0) free.push_back(b);
  }

  // kv.rs:85-121. Returns 0, 1 (full) or 2 (non-contiguous).
  // The copy-on-write body of kv.rs:99-110: every layer's K and V rows of
  // block src copied into block dst (copy_within).
  void copy_block(size_t src_b, size_t dst_b) {
    const size_t n = kBlock * kv_dim * elem;
    for (size_t l = 0; l < n_layers; ++l) {
      const size_t src = offset(l, src_b, 0) * elem, dst = offset(l, dst_b, 0) * elem;
      std::memmove(&k[dst], &k[src], n);
      std::memmove(&v[dst], &v[src], n);
      if (elem == 1) {  // the block's scales travel with its quants
        const size_t ns = kBlock * kv_dim / 32, s0 = offset(l, src_b, 0) / 32, d0 = offset(l, dst_b, 0) / 32;
        std::memmove(&ks[d0], &ks[s0], ns * 2);
        std::memmove(&vs[d0], &vs[s0], ns * 2);
      }
    }
  }

  int append(uint32_t seq, size_t pos, size_t *block_out, size_t *slot_out) {
    Seq &s = seqs[seq];  // entry().or_default()
    if (pos != s.len) {
      err = "seq " + std::to_string(seq) + ": position " + std::to_string(pos) +
            " is not contiguous (length " + std::to_string(s.len) + ")";
      return 2;
    }
    const size_t slot = pos % kBlock;
    if (slot == 0) {
      size_t b;
      if (!alloc(&b)) return 1;
      s.blocks.push_back(b);
    } else {
      const size_t last = s.blocks.back();
      if (refs[last] > 1) {
        size_t nb;
        if (!alloc(&nb)) return 1;
        copy_block(last, nb);
        release(last);
        s.blocks.back() = nb;
        ++cow_copies;
      }
    }
    s.len = pos + 1;
    *block_out = s.blocks.back();
    *slot_out = slot;
    return 0;
  }

  void write(size_t layer, size_t block, size_t slot, const float *kr, const float *vr) {
    const size_t o = offset(layer, block, slot) * elem;  // kv.rs:123-131
    if (elem == 2) {
      narrow_row(kr, (uint16_t *)&k[o], kv_dim);
      narrow_row(vr, (uint16_t *)&v[o], kv_dim);
    } else if (elem == 1) {
      for (size_t b = 0; b < kv_dim / 32; ++b) {
        ks[o / 32 + b] = f32_to_f16(quantize_block(kr + 32 * b, (int8_t *)&k[o + 32 * b]));
        vs[o / 32 + b] = f32_to_f16(quantize_block(vr + 32 * b, (int8_t *)&v[o + 32 * b]));
      }
    } else {
      std::memcpy(&k[o], kr, kv_dim * 4);
      std::memcpy(&v[o], vr, kv_dim * 4);
    }
  }

  // Q8_0 row read back as d * q (quant.rs:188-193); o = the row's byte offset.
  void dequant(const std::vector<uint8_t> &pool, const std::vector<uint16_t> &sc, size_t o, size_t col,
               size_t n, float *dst) const {
    for (size_t i = 0; i < n; ++i)
      dst[i] = f16_to_f32(sc[(o + col + i) / 32]) * (float)(int8_t)pool[o + col + i];
  }

  // Byte offset of position p of a sequence's table (kv.rs:146-148).
  size_t row_offset(size_t layer, const std::vector<size_t> &blocks, size_t p) const {
    return offset(layer, blocks[p / kBlock], p % kBlock) * elem;
  }

  void truncate(uint32_t seq, size_t from) {  // kv.rs:153-169
    auto it = seqs.find(seq);
    if (it == seqs.end()) return;
    Seq s = std::move(it->second);
    seqs.erase(it);
    if (from >= s.len) {
      seqs[seq] = std::move(s);
      return;
    }
    const size_t keep = (from + kBlock - 1) / kBlock;
    for (size_t i = keep; i < s.blocks.size(); ++i) release(s.blocks[i]);
    s.blocks.resize(keep);
    s.len = from;
    if (from > 0) seqs[seq] = std::move(s);
  }

  void share(uint32_t src, uint32_t dst, size_t len) {  // kv.rs:172-183
    truncate(dst, 0);
    auto it = seqs.find(src);
    if (it == seqs.end()) return;
    len = std::min(len, it->second.len);
    std::vector<size_t> blocks(it->second.blocks.begin(),
                               it->second.blocks.begin() + (len + kBlock - 1) / kBlock);
    for (size_t b : blocks) refs[b] += 1;
    if (len > 0) seqs[dst] = Seq{std::move(blocks), len};
  }

  size_t len(uint32_t seq) const {
    auto it = seqs.find(seq);
    return it == seqs.end() ? 0 : it->second.len;
  }
};

// dot() of model.rs:158-172: 8 partial sums over chunks_exact(8), sequential
// tail, then acc summed left to right plus the tail. Built without FMA
// contraction, so each step is a rounded multiply then a rounded add.
inline float dot8(const float *a, const float *b, size_t n) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  const size_t nc = n / 8 * 8;
  for (size_t i = 0; i < nc; i += 8)
    for (int j = 0; j < 8; ++j) acc[j] += a[i + j] * b[i + j];
  float tail = -0.0f;  // f32 Sum starts from -0.0
  for (size_t i = nc; i < n; ++i) tail += a[i] * b[i];
  float s = -0.0f;
  for (int j = 0; j < 8; ++j) s += acc[j];
  return s + tail;
}

struct Scratch {
  std::vector<float> scores, row;
};

// The attention closure of model.rs:435-474 for task idx = i*n_kv_heads+kvh.
void attention_task(const OracleKv &kv, size_t layer, const std::vector<size_t> &blocks,
                    size_t len, const float *qs, size_t group, size_t hd, size_t kvh, float scale,
                    float *out, Scratch &sc) {
  std::vector<float> &scores = sc.scores, &row = sc.row;
  scores.assign(group * len, 0.0f);
  row.resize(hd);
  const size_t col = kvh * hd * kv.elem;
  for (size_t p = 0; p < len; ++p) {  // K pass
    const uint8_t *kr = kv.k.data() + kv.row_offset(layer, blocks, p) + col;
    if (kv.elem == 2)
      widen_row((const uint16_t *)kr, row.data(), hd);
    else if (kv.elem == 1)
      kv.dequant(kv.k, kv.ks, kv.row_offset(layer, blocks, p), col, hd, row.data());
    else
      std::memcpy(row.data(), kr, hd * 4);
    for (size_t g = 0; g < group; ++g) scores[g * len + p] = dot8(qs + g * hd, row.data(), hd) * scale;
  }
  for (size_t g = 0; g < group; ++g) {  // softmax per query head
    float *sg = scores.data() + g * len;
    float mx = -INFINITY;
    for (size_t p = 0; p < len; ++p) mx = std::fmax(mx, sg[p]);
    float sum = 0.0f;
    for (size_t p = 0; p < len; ++p) {
      sg[p] = std::exp(sg[p] - mx);  // f32::exp -> libm expf
      sum += sg[p];
    }
    const float inv = 1.0f / sum;
    for (size_t p = 0; p < len; ++p) sg[p] *= inv;
  }
  std::fill(out, out + group * hd, 0.0f);
  for (size_t p = 0; p < len; ++p) {  // V pass
    const uint8_t *vr = kv.v.data() + kv.row_offset(layer, blocks, p) + col;
    if (kv.elem == 2)
      widen_row((const uint16_t *)vr, row.data(), hd);
    else if (kv.elem == 1)
      kv.dequant(kv.v, kv.vs, kv.row_offset(layer, blocks, p), col, hd, row.data());
    else
      std::memcpy(row.data(), vr, hd * 4);
    for (size_t g = 0; g < group; ++g) {
      const float w = scores[g * len + p];
      float *o = out + g * hd;
      for (size_t j = 0; j < hd; ++j) o[j] += w * row[j];
    }
  }
}

thread_local std::string g_err;

// One pool per thread count, kept until exit, so a pool is never destroyed
// while another caller uses it.
std::mutex g_pool_mu;
std::unordered_map<size_t, Pool *> g_pools;

Pool &pool_for(size_t threads) {
  if (threads == 0) threads = 1;
  std::lock_guard<std::mutex> g(g_pool_mu);
  Pool *&p = g_pools[threads];
  if (!p) p = new Pool(threads);
  return *p;
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI used by the Python test and bench harness (ctypes).
// ---------------------------------------------------------------------------
extern "C" {

const char *ora_last_error(void) { return g_err.c_str(); }

void ora_f32_to_f16(const float *src, uint16_t *dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = f32_to_f16(src[i]);
}
void ora_f32_to_f16_simd(const float *src, uint16_t *dst, size_t n) { narrow_row(src, dst, n); }
void ora_f16_to_f32(const uint16_t *src, float *dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = f16_to_f32(src[i]);
}
void ora_f16_to_f32_simd(const uint16_t *src, float *dst, size_t n) { widen_row(src, dst, n); }
int ora_has_f16c(void) {
#if defined(__F16C__)
  return 1;
#else
  return 0;
#endif
}

// dtype 0 = f16, 1 = f32, 2 = Q8_0 (kv_dim a multiple of 32).
void *ora_create(size_t n_layers, size_t kv_dim, size_t n_tokens, int dtype) {
  if (kv_dim == 0 || n_layers == 0 || dtype < 0 || dtype > 2) return nullptr;
  if (dtype == 2 && kv_dim % 32 != 0) return nullptr;
  return new OracleKv(n_layers, kv_dim, n_tokens, dtype == 0 ? 2 : dtype == 1 ? 4 : 1);
}

// quant.rs:785-791 on one 32-element block: quants to q, returns d (f32).
float ora_quantize_block(const float *x, int8_t *q) { return quantize_block(x, q); }
void ora_destroy(void *h) { delete (OracleKv *)h; }

size_t ora_capacity(void *h) { return ((OracleKv *)h)->n_blocks * kBlock; }
size_t ora_bytes(void *h) {
  auto *kv = (OracleKv *)h;
  return kv->k.size() + kv->v.size() + 2 * (kv->ks.size() + kv->vs.size());
}
size_t ora_n_blocks(void *h) { return ((OracleKv *)h)->n_blocks; }
size_t ora_len(void *h, uint32_t seq) { return ((OracleKv *)h)->len(seq); }
size_t ora_free_blocks(void *h) { return ((OracleKv *)h)->free.size(); }
uint32_t ora_refcount(void *h, size_t block) { return ((OracleKv *)h)->refs[block]; }
uint64_t ora_cow_copies(void *h) { return ((OracleKv *)h)->cow_copies; }
int ora_has_seq(void *h, uint32_t seq) {
  auto *kv = (OracleKv *)h;
  return kv->seqs.count(seq) ? 1 : 0;
}

// Seed the free stack so that successive allocations return order[0],
// order[1], ... (harness hook for randomised block tables).
int ora_init_free_order(void *h, const uint32_t *order, size_t n) {
  auto *kv = (OracleKv *)h;
  if (n != kv->n_blocks || !kv->seqs.empty()) return 5;
  kv->free.clear();
  for (size_t i = n; i-- > 0;) kv->free.push_back(order[i]);
  return 0;
}

int ora_append(void *h, uint32_t seq, size_t pos, uint32_t *block, uint32_t *slot) {
  auto *kv = (OracleKv *)h;
  size_t b = 0, s = 0;
  const int rc = kv->append(seq, pos, &b, &s);
  if (rc) {
    g_err = kv->err;
    return rc;
  }
  *block = (uint32_t)b;
  *slot = (uint32_t)s;
  return 0;
}

// model.rs:380-383: claim cells for a whole batch in order; stops at the
// first error (earlier claims stay, as with collect::<Result<_>>()).
int ora_append_batch(void *h, size_t n, const uint32_t *seqs, const uint64_t *pos,
                     int32_t *slot_mapping, size_t *n_done) {
  auto *kv = (OracleKv *)h;
  for (size_t i = 0; i < n; ++i) {
    size_t b = 0, s = 0;
    const int rc = kv->append(seqs[i], (size_t)pos[i], &b, &s);
    if (rc) {
      g_err = kv->err;
      if (n_done) *n_done = i;
      return rc;
    }
    slot_mapping[i] = (int32_t)(b * kBlock + s);
  }
  if (n_done) *n_done = n;
  return 0;
}

void ora_write(void *h, size_t layer, size_t block, size_t slot, const float *k, const float *v) {
  ((OracleKv *)h)->write(layer, block, slot, k, v);
}

// model.rs:414-429 for a batch: write row i to its claimed cell (slot mapping
// entry block*16+slot; negative entries are skipped).
void ora_write_batch(void *h, size_t layer, size_t n, const int32_t *slot_mapping, const float *k,
                     const float *v) {
  auto *kv = (OracleKv *)h;
  for (size_t i = 0; i < n; ++i) {
    if (slot_mapping[i] < 0) continue;
    kv->write(layer, (size_t)slot_mapping[i] / kBlock, (size_t)slot_mapping[i] % kBlock,
              k + i * kv->kv_dim, v + i * kv->kv_dim);
  }
}

// Model::rope (model.rs:291-308) with inv_freq of model.rs:263-265: per head,
// pair i rotates (v[a], v[b]) by pos * inv_freq[i], a/b = (i, i + rope_dim/2)
// for NeoX models, else (2i, 2i + 1); (sin, cos) = f32::sin_cos, i.e. libm
// sinf/cosf; no fused multiply-add (built with -ffp-contract=off).
static void rope(float *x, size_t n_heads, size_t head_dim, size_t rope_dim, bool neox,
                 const std::vector<float> &inv_freq, size_t pos) {
  const size_t half = rope_dim / 2;
  for (size_t h = 0; h < n_heads; ++h) {
    float *v = x + h * head_dim;
    for (size_t i = 0; i < inv_freq.size(); ++i) {
      const float ang = (float)pos * inv_freq[i];
      const float sn = sinf(ang), cs = cosf(ang);
      const size_t a = neox ? i : 2 * i, b = neox ? i + half : 2 * i + 1;
      const float x0 = v[a], x1 = v[b];
      v[a] = x0 * cs - x1 * sn;
      v[b] = x0 * sn + x1 * cs;
    }
  }
}

static std::vector<float> rope_inv_freq(float base, size_t rope_dim) {
  std::vector<float> inv(rope_dim / 2);
  for (size_t i = 0; i < inv.size(); ++i) inv[i] = powf(base, -2.0f * (float)i / (float)rope_dim);
  return inv;
}

// The per-token body of model.rs:414-429: RoPE on the token's q (n_heads
// heads, in place, when q is not null) and k (the cache's kv heads), then
// write(layer, block, slot, k, v). Rows are kv_dim (k, v) / q_stride (q) apart.
void ora_write_rope_batch(void *h, size_t layer, size_t n, const int32_t *slot_mapping,
                          const int32_t *positions, const float *k, const float *v, float *q,
                          size_t q_stride, size_t n_heads, float base, size_t rope_dim,
                          size_t head_dim, int neox) {
  auto *kv = (OracleKv *)h;
  const std::vector<float> inv = rope_inv_freq(base, rope_dim);
  std::vector<float> kr(kv->kv_dim);
  for (size_t i = 0; i < n; ++i) {
    const size_t pos = (size_t)positions[i];
    if (q) rope(q + i * q_stride, n_heads, head_dim, rope_dim, neox != 0, inv, pos);
    if (slot_mapping[i] < 0) continue;
    std::copy(k + i * kv->kv_dim, k + (i + 1) * kv->kv_dim, kr.begin());
    rope(kr.data(), kv->kv_dim / head_dim, head_dim, rope_dim, neox != 0, inv, pos);
    kv->write(layer, (size_t)slot_mapping[i] / kBlock, (size_t)slot_mapping[i] % kBlock, kr.data(),
              v + i * kv->kv_dim);
  }
}

// rows(layer, seq, n) collected into contiguous [n][kv_dim] buffers (kv.rs:133-150).
int ora_rows(void *h, size_t layer, uint32_t seq, size_t n, void *k_out, void *v_out) {
  auto *kv = (OracleKv *)h;
  auto it = kv->seqs.find(seq);
  static const std::vector<size_t> empty;
  const std::vector<size_t> &blocks = it == kv->seqs.end() ? empty : it->second.blocks;
  if ((n + kBlock - 1) / kBlock > blocks.size()) {
    g_err = "index out of range";
    return 3;
  }
  const size_t row = kv->kv_dim * kv->elem;
  for (size_t p = 0; p < n; ++p) {
    const size_t o = kv->row_offset(layer, blocks, p);
    std::memcpy((uint8_t *)k_out + p * row, &kv->k[o], row);
    std::memcpy((uint8_t *)v_out + p * row, &kv->v[o], row);
  }
  return 0;
}

int ora_block_table(void *h, uint32_t seq, int32_t *out, size_t cap, size_t *n_blocks) {
  auto *kv = (OracleKv *)h;
  auto it = kv->seqs.find(seq);
  const size_t nb = it == kv->seqs.end() ? 0 : it->second.blocks.size();
  if (n_blocks) *n_blocks = nb;
  if (nb > cap) return 3;
  for (size_t i = 0; i < nb; ++i) out[i] = (int32_t)it->second.blocks[i];
  return 0;
}

void ora_truncate(void *h, uint32_t seq, size_t from) { ((OracleKv *)h)->truncate(seq, from); }

// The copy-on-write body (kv.rs:99-110) for n (src, dst) block pairs, in
// order; pairs with a block out of range are skipped. Returns pairs copied.
size_t ora_copy_blocks(void *h, size_t n, const int32_t *pairs) {
  auto *kv = (OracleKv *)h;
  size_t done = 0;
  for (size_t i = 0; i < n; ++i) {
    const int32_t a = pairs[2 * i], b = pairs[2 * i + 1];
    if (a < 0 || b < 0 || (size_t)a >= kv->n_blocks || (size_t)b >= kv->n_blocks) continue;
    kv->copy_block((size_t)a, (size_t)b);
    ++done;
  }
  return done;
}
void ora_share(void *h, uint32_t src, uint32_t dst, size_t len) {
  ((OracleKv *)h)->share(src, dst, len);
}

// Raw pool bytes of one layer (reference layout [block][slot][kv_dim]).
void ora_pool(void *h, size_t layer, void *k_out, void *v_out) {
  auto *kv = (OracleKv *)h;
  const size_t n = kv->n_blocks * kBlock * kv->kv_dim * kv->elem;
  std::memcpy(k_out, &kv->k[layer * n], n);
  std::memcpy(v_out, &kv->v[layer * n], n);
}

// Replace one layer's raw pool bytes (same layout as ora_pool), so the
// oracle can run on exactly the state another implementation produced.
void ora_load_pool(void *h, size_t layer, const void *k_in, const void *v_in) {
  auto *kv = (OracleKv *)h;
  const size_t n = kv->n_blocks * kBlock * kv->kv_dim * kv->elem;
  std::memcpy(&kv->k[layer * n], k_in, n);
  std::memcpy(&kv->v[layer * n], v_in, n);
}

// Q8_0 scale pools of one layer ([block][slot][kv_dim/32] f16 bits), read or
// replaced like ora_pool / ora_load_pool.
int ora_scales(void *h, size_t layer, uint16_t *k_out, uint16_t *v_out) {
  auto *kv = (OracleKv *)h;
  if (kv->elem != 1) return 5;
  const size_t n = kv->n_blocks * kBlock * kv->kv_dim / 32;
  std::memcpy(k_out, &kv->ks[layer * n], n * 2);
  std::memcpy(v_out, &kv->vs[layer * n], n * 2);
  return 0;
}
int ora_load_scales(void *h, size_t layer, const uint16_t *k_in, const uint16_t *v_in) {
  auto *kv = (OracleKv *)h;
  if (kv->elem != 1) return 5;
  const size_t n = kv->n_blocks * kBlock * kv->kv_dim / 32;
  std::memcpy(&kv->ks[layer * n], k_in, n * 2);
  std::memcpy(&kv->vs[layer * n], v_in, n * 2);
  return 0;
}

// Attention over the cache (model.rs:431-475) for n tokens of a batch:
// token i belongs to seqs[i] at positions[i]; q and out are [n][n_heads*head_dim].
int ora_attention(void *h, size_t layer, size_t n, const uint32_t *seqs, const uint64_t *positions,
                  size_t n_heads, size_t head_dim, float scale, const float *q, float *out,
                  size_t threads) {
  auto *kv = (OracleKv *)h;
  if (head_dim == 0 || kv->kv_dim % head_dim != 0) return 5;
  const size_t n_kv_heads = kv->kv_dim / head_dim;
  if (n_heads % n_kv_heads != 0) return 5;
  const size_t group = n_heads / n_kv_heads, q_dim = n_heads * head_dim;
  std::vector<const std::vector<size_t> *> tables(n);
  static const std::vector<size_t> empty;
  for (size_t i = 0; i < n; ++i) {
    auto it = kv->seqs.find(seqs[i]);
    tables[i] = it == kv->seqs.end() ? &empty : &it->second.blocks;
    if ((positions[i] + 1 + kBlock - 1) / kBlock > tables[i]->size()) return 3;
  }
  Pool &pool = pool_for(threads);
  const std::function<void(size_t)> task = [&](size_t idx) {
    thread_local Scratch sc;
    const size_t i = idx / n_kv_heads, kvh = idx % n_kv_heads;
    attention_task(*kv, layer, *tables[i], (size_t)positions[i] + 1,
                   q + i * q_dim + kvh * group * head_dim, group, head_dim, kvh, scale,
                   out + i * q_dim + kvh * group * head_dim, sc);
  };
  pool.run(n * n_kv_heads, task);
  return 0;
}

// Same attention with the queries' contexts given as explicit block tables
// and lengths, i.e. the kernel-level interface (tables[i*stride + j]).
int ora_attention_tables(void *h, size_t layer, size_t n, const int32_t *tables_in, size_t stride,
                         const int32_t *lens, size_t n_heads, size_t head_dim, float scale,
                         const float *q, float *out, size_t threads) {
  auto *kv = (OracleKv *)h;
  if (head_dim == 0 || kv->kv_dim % head_dim != 0) return 5;
  const size_t n_kv_heads = kv->kv_dim / head_dim;
  if (n_heads % n_kv_heads != 0) return 5;
  const size_t group = n_heads / n_kv_heads, q_dim = n_heads * head_dim;
  std::vector<std::vector<size_t>> tables(n);
  for (size_t i = 0; i < n; ++i) {
    const size_t nb = ((size_t)lens[i] + kBlock - 1) / kBlock;
    if (nb > stride) return 3;
    for (size_t j = 0; j < nb; ++j) {
      if (tables_in[i * stride + j] < 0 || (size_t)tables_in[i * stride + j] >= kv->n_blocks) return 3;
      tables[i].push_back((size_t)tables_in[i * stride + j]);
    }
  }
  Pool &pool = pool_for(threads);
  const std::function<void(size_t)> task = [&](size_t idx) {
    thread_local Scratch sc;
    const size_t i = idx / n_kv_heads, kvh = idx % n_kv_heads;
    attention_task(*kv, layer, tables[i], (size_t)lens[i], q + i * q_dim + kvh * group * head_dim,
                   group, head_dim, kvh, scale, out + i * q_dim + kvh * group * head_dim, sc);
  };
  pool.run(n * n_kv_heads, task);
  return 0;
}

// Pool exercise matching pool.rs's tests: run n tasks that each add i to a
// counter slot; returns the number of tasks that ran (exactly-once check).
uint64_t ora_pool_selftest(size_t threads, size_t n, uint32_t *hits) {
  Pool &pool = pool_for(threads);
  std::vector<std::atomic<uint32_t>> h(n);
  const std::function<void(size_t)> task = [&](size_t i) { h[i].fetch_add(1); };
  pool.run(n, task);
  uint64_t total = 0;
  for (size_t i = 0; i < n; ++i) {
    hits[i] = h[i].load();
    total += hits[i];
  }
  return total;
}

}  // extern "C"
