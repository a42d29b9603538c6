//! FFI to libltkv.so, the MI355X paged KV cache (`include/ltkv.h`), and a safe
//! `KvCache` with the method set of `langtrain_native::kv::KvCache`
//! (engine/crates/native/src/kv.rs:34-188), so `NativeBackend`
//! (engine/crates/native/src/lib.rs:45-198) can swap its cache type.
//!
//! `ffi` declares every entry point of the header one to one (the repository's
//! tests/test_rust_binding.py checks names, argument and return types against
//! the header). `KvCache` wraps the host-side methods; device operations take
//! raw device pointers and stay `unsafe`: the caller guarantees that they point
//! to device memory of the stated sizes, valid on the cache's stream.
#![allow(non_camel_case_types)]

use std::ffi::{c_char, c_int, c_uint, c_void, CStr};

pub mod ffi {
    use super::*;

    #[repr(C)]
    pub struct ltkv_cache {
        _p: [u8; 0],
    }

    pub const LTKV_BLOCK: usize = 16;
    pub const LTKV_OK: c_int = 0;
    pub const LTKV_ERR_FULL: c_int = 1;
    pub const LTKV_ERR_NONCONTIG: c_int = 2;
    pub const LTKV_ERR_RANGE: c_int = 3;
    pub const LTKV_ERR_HIP: c_int = 4;
    pub const LTKV_ERR_ARG: c_int = 5;
    pub const LTKV_NO_DEVICE: c_int = -1;
    pub const LTKV_F16: c_int = 0;
    pub const LTKV_F32: c_int = 1;
    pub const LTKV_Q8_0: c_int = 2;
    pub const LTKV_PLAN_SHARED_PREFIX: c_uint = 1;
    pub const LTKV_PLAN_F16_PRODUCTS: c_uint = 2;
    pub const LTKV_NOALLOC_SCRATCH_BYTES: usize = 32 << 20;
    pub const LTKV_ENGINE_AUTO: c_int = 0;
    pub const LTKV_ENGINE_VALU: c_int = 1;

    #[link(name = "ltkv")]
    extern "C" {
        pub fn ltkv_last_error() -> *const c_char;

        // lifecycle
        pub fn ltkv_create(n_layers: usize, kv_dim: usize, n_tokens: usize, dtype: c_int, device: c_int,
                           out: *mut *mut ltkv_cache) -> c_int;
        pub fn ltkv_destroy(c: *mut ltkv_cache);
        pub fn ltkv_set_stream(c: *mut ltkv_cache, hip_stream: *mut c_void) -> c_int;

        // queries (kv.rs:50-60,185-187)
        pub fn ltkv_capacity(c: *const ltkv_cache) -> usize;
        pub fn ltkv_bytes(c: *const ltkv_cache) -> usize;
        pub fn ltkv_len(c: *const ltkv_cache, seq: u32) -> usize;
        pub fn ltkv_free_blocks(c: *const ltkv_cache) -> usize;
        pub fn ltkv_n_blocks(c: *const ltkv_cache) -> usize;
        pub fn ltkv_kv_dim(c: *const ltkv_cache) -> usize;
        pub fn ltkv_refcount(c: *const ltkv_cache, block: u32) -> u32;
        pub fn ltkv_cow_copies(c: *const ltkv_cache) -> u64;

        // block management
        pub fn ltkv_append(c: *mut ltkv_cache, seq: u32, pos: usize, block: *mut u32, slot: *mut u32) -> c_int;
        pub fn ltkv_append_batch(c: *mut ltkv_cache, n: usize, seqs: *const u32, pos: *const u64,
                                 slot_mapping: *mut i32, n_done: *mut usize) -> c_int;
        pub fn ltkv_truncate(c: *mut ltkv_cache, seq: u32, from: usize);
        pub fn ltkv_share(c: *mut ltkv_cache, src: u32, dst: u32, len: usize);
        pub fn ltkv_block_table(c: *const ltkv_cache, seq: u32, out: *mut i32, cap: usize,
                                n_blocks: *mut usize) -> c_int;
        pub fn ltkv_block_tables(c: *const ltkv_cache, n: usize, seqs: *const u32, out: *mut i32,
                                 stride: usize) -> c_int;
        pub fn ltkv_init_free_order(c: *mut ltkv_cache, order: *const u32, n: usize) -> c_int;

        // device ops (enqueued on the cache's stream)
        pub fn ltkv_write(c: *mut ltkv_cache, layer: usize, n: usize, d_slot_mapping: *const i32,
                          d_k: *const f32, d_v: *const f32, src_stride: usize) -> c_int;
        pub fn ltkv_cell_order(c: *const ltkv_cache, n: usize, slot_mapping: *const i32, order: *mut i32,
                               m: *mut usize) -> c_int;
        pub fn ltkv_write_ordered(c: *mut ltkv_cache, layer: usize, n: usize, d_slot_mapping: *const i32,
                                  d_k: *const f32, d_v: *const f32, src_stride: usize, m: usize,
                                  d_order: *const i32) -> c_int;
        pub fn ltkv_rope_init(c: *mut ltkv_cache, base: f32, rope_dim: usize, head_dim: usize, neox: c_int,
                              max_positions: usize) -> c_int;
        pub fn ltkv_write_rope(c: *mut ltkv_cache, layer: usize, n: usize, d_slot_mapping: *const i32,
                               d_positions: *const i32, d_k: *const f32, d_v: *const f32, src_stride: usize,
                               d_q: *mut f32, q_stride: usize, n_heads: usize) -> c_int;
        pub fn ltkv_copy_blocks(c: *mut ltkv_cache, n: usize, d_pairs: *const i32) -> c_int;
        pub fn ltkv_gather(c: *mut ltkv_cache, layer: usize, n: usize, d_tables: *const i32, table_stride: usize,
                           d_lens: *const i32, d_out_offsets: *const i64, d_k_out: *mut c_void,
                           d_v_out: *mut c_void) -> c_int;
        pub fn ltkv_decode_attention(c: *mut ltkv_cache, layer: usize, n: usize, n_heads: usize, head_dim: usize,
                                     scale: f32, d_q: *const f32, d_tables: *const i32, table_stride: usize,
                                     d_lens: *const i32, d_out: *mut f32) -> c_int;
        pub fn ltkv_decode_attention_noalloc(c: *mut ltkv_cache, layer: usize, n: usize, n_heads: usize,
                                             head_dim: usize, scale: f32, d_q: *const f32, d_tables: *const i32,
                                             table_stride: usize, d_lens: *const i32, d_out: *mut f32) -> c_int;
        pub fn ltkv_append_decode_attention(c: *mut ltkv_cache, layer: usize, n: usize, n_heads: usize,
                                            head_dim: usize, scale: f32, d_q: *const f32, d_tables: *const i32,
                                            table_stride: usize, d_lens: *const i32, d_slot_mapping: *const i32,
                                            d_k: *const f32, d_v: *const f32, src_stride: usize,
                                            d_out: *mut f32) -> c_int;
        pub fn ltkv_set_attention_partition(c: *mut ltkv_cache, tokens: usize) -> c_int;
        pub fn ltkv_set_attention_engine(c: *mut ltkv_cache, engine: c_int) -> c_int;

        // planned attention
        pub fn ltkv_plan_attention(c: *mut ltkv_cache, n: usize, seqs: *const u32, lens: *const u32,
                                   n_heads: usize, head_dim: usize, flags: c_uint) -> c_int;
        pub fn ltkv_planned_attention(c: *mut ltkv_cache, layer: usize, scale: f32, d_q: *const f32,
                                      d_out: *mut f32) -> c_int;
        pub fn ltkv_plan_stats(c: *const ltkv_cache, out: *mut u64) -> c_int;

        // resident block tables
        pub fn ltkv_seq_rows(c: *const ltkv_cache, n: usize, seqs: *const u32, rows_out: *mut i32) -> c_int;
        pub fn ltkv_sync_tables(c: *mut ltkv_cache) -> c_int;
        pub fn ltkv_resident_tables(c: *mut ltkv_cache, d_tables: *mut *const i32, d_lengths: *mut *const i32,
                                    stride: *mut usize, n_rows: *mut usize) -> c_int;
        pub fn ltkv_slot_mapping(c: *mut ltkv_cache, n: usize, d_rows: *const i32, d_pos: *const i64,
                                 d_slot_mapping: *mut i32) -> c_int;
        pub fn ltkv_decode_attention_rows(c: *mut ltkv_cache, layer: usize, n: usize, n_heads: usize,
                                          head_dim: usize, scale: f32, d_q: *const f32, d_rows: *const i32,
                                          d_lens: *const i32, d_out: *mut f32) -> c_int;
        pub fn ltkv_table_uploads(c: *const ltkv_cache, entries: *mut u64) -> c_int;

        // host conveniences
        pub fn ltkv_read_resident_tables(c: *mut ltkv_cache, h_tables: *mut i32, h_lengths: *mut i32) -> c_int;
        pub fn ltkv_read_pool(c: *mut ltkv_cache, layer: usize, h_k: *mut c_void, h_v: *mut c_void) -> c_int;
        pub fn ltkv_read_scales(c: *mut ltkv_cache, layer: usize, h_k: *mut u16, h_v: *mut u16) -> c_int;
        pub fn ltkv_rows(c: *mut ltkv_cache, layer: usize, seq: u32, n: usize, h_k: *mut c_void,
                         h_v: *mut c_void) -> c_int;
        pub fn ltkv_write_row(c: *mut ltkv_cache, layer: usize, block: u32, slot: u32, h_k: *const f32,
                              h_v: *const f32) -> c_int;
        pub fn ltkv_synchronize(c: *mut ltkv_cache) -> c_int;
    }
}

use ffi::*;

/// Element type of the pools: `F16` is the reference's (kv.rs:5-6).
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum Dtype {
    F16,
    F32,
    Q8_0,
}

/// An error returned by the C ABI: its `LTKV_ERR_*` code and the library's
/// message (the reference's texts for "KV cache full", kv.rs:71, and the
/// non-contiguous append, kv.rs:88-91).
#[derive(Debug, Clone)]
pub struct Error {
    pub code: c_int,
    pub message: String,
}

impl std::fmt::Display for Error {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        f.write_str(&self.message)
    }
}

impl std::error::Error for Error {}

fn check(rc: c_int) -> anyhow::Result<()> {
    if rc == LTKV_OK {
        return Ok(());
    }
    let message = unsafe {
        let p = ltkv_last_error();
        if p.is_null() { String::new() } else { CStr::from_ptr(p).to_string_lossy().into_owned() }
    };
    Err(Error { code: rc, message }.into())
}

/// The paged KV cache on one HIP device: kv.rs's `KvCache` with its K/V pools
/// in HBM. One thread mutates it at a time (`&mut self`), as in the engine.
pub struct KvCache {
    raw: *mut ltkv_cache,
    /// kv.rs:18 `pub kv_dim`.
    pub kv_dim: usize,
    dtype: Dtype,
}

// The handle is owned by one engine thread at a time (scheduler.rs:103-114).
unsafe impl Send for KvCache {}

impl Drop for KvCache {
    fn drop(&mut self) {
        unsafe { ltkv_destroy(self.raw) }
    }
}

impl KvCache {
    /// KvCache::new(n_layers, kv_dim, n_tokens) (kv.rs:35-48) on HIP device
    /// `device` (or `LTKV_NO_DEVICE` for the allocator alone).
    pub fn new(n_layers: usize, kv_dim: usize, n_tokens: usize, dtype: Dtype, device: c_int) -> anyhow::Result<Self> {
        let code = match dtype {
            Dtype::F16 => LTKV_F16,
            Dtype::F32 => LTKV_F32,
            Dtype::Q8_0 => LTKV_Q8_0,
        };
        let mut raw = std::ptr::null_mut();
        check(unsafe { ltkv_create(n_layers, kv_dim, n_tokens, code, device, &mut raw) })?;
        Ok(Self { raw, kv_dim, dtype })
    }

    pub fn dtype(&self) -> Dtype {
        self.dtype
    }

    pub fn as_raw(&self) -> *mut ltkv_cache {
        self.raw
    }

    /// Stream (a `hipStream_t`) on which every device op of this cache is enqueued.
    pub fn set_stream(&mut self, stream: *mut c_void) -> anyhow::Result<()> {
        check(unsafe { ltkv_set_stream(self.raw, stream) })
    }

    pub fn capacity(&self) -> usize {
        unsafe { ltkv_capacity(self.raw) }
    }

    pub fn bytes(&self) -> usize {
        unsafe { ltkv_bytes(self.raw) }
    }

    pub fn len(&self, seq: u32) -> usize {
        unsafe { ltkv_len(self.raw, seq) }
    }

    pub fn free_blocks(&self) -> usize {
        unsafe { ltkv_free_blocks(self.raw) }
    }

    pub fn n_blocks(&self) -> usize {
        unsafe { ltkv_n_blocks(self.raw) }
    }

    pub fn refcount(&self, block: u32) -> u32 {
        unsafe { ltkv_refcount(self.raw, block) }
    }

    pub fn cow_copies(&self) -> u64 {
        unsafe { ltkv_cow_copies(self.raw) }
    }

    /// kv.rs:85-121: the cell for `pos` (which must equal `len(seq)`).
    pub fn append(&mut self, seq: u32, pos: usize) -> anyhow::Result<(usize, usize)> {
        let (mut block, mut slot) = (0u32, 0u32);
        check(unsafe { ltkv_append(self.raw, seq, pos, &mut block, &mut slot) })?;
        Ok((block as usize, slot as usize))
    }

    /// The claim of model.rs:380-383 for a whole batch: slot_mapping[i] =
    /// block * 16 + slot of (seqs[i], pos[i]). On error the claims before the
    /// failing entry stay made, as `collect::<Result<_>>()?` leaves them.
    pub fn append_batch(&mut self, seqs: &[u32], pos: &[u64], slot_mapping: &mut [i32]) -> anyhow::Result<()> {
        anyhow::ensure!(seqs.len() == pos.len() && slot_mapping.len() >= seqs.len(), "batch arrays differ in length");
        let mut done = 0usize;
        check(unsafe {
            ltkv_append_batch(self.raw, seqs.len(), seqs.as_ptr(), pos.as_ptr(), slot_mapping.as_mut_ptr(), &mut done)
        })
    }

    /// kv.rs:123-131 from host rows: the f32 rows of K and V into (block,
    /// slot) of `layer`. The reference panics on a bad cell; this returns the
    /// library's error.
    pub fn write(&mut self, layer: usize, block: usize, slot: usize, k: &[f32], v: &[f32]) -> anyhow::Result<()> {
        anyhow::ensure!(k.len() == self.kv_dim && v.len() == self.kv_dim, "rows must hold kv_dim values");
        let block = u32::try_from(block)?;
        let slot = u32::try_from(slot)?;
        check(unsafe { ltkv_write_row(self.raw, layer, block, slot, k.as_ptr(), v.as_ptr()) })
    }

    /// kv.rs:133-150 collected: the first `n` K and V rows of `seq` (f16 bits)
    /// of an F16 cache (`rows_f32` for an F32 cache; Q8_0 has no rows form).
    pub fn rows(&mut self, layer: usize, seq: u32, n: usize) -> anyhow::Result<(Vec<u16>, Vec<u16>)> {
        anyhow::ensure!(self.dtype == Dtype::F16, "rows gives f16 rows: the cache holds {:?}", self.dtype);
        let mut k = vec![0u16; n * self.kv_dim];
        let mut v = vec![0u16; n * self.kv_dim];
        check(unsafe { ltkv_rows(self.raw, layer, seq, n, k.as_mut_ptr().cast(), v.as_mut_ptr().cast()) })?;
        Ok((k, v))
    }

    /// The first `n` K and V rows of `seq` of an F32 cache.
    pub fn rows_f32(&mut self, layer: usize, seq: u32, n: usize) -> anyhow::Result<(Vec<f32>, Vec<f32>)> {
        anyhow::ensure!(self.dtype == Dtype::F32, "rows_f32 gives f32 rows: the cache holds {:?}", self.dtype);
        let mut k = vec![0f32; n * self.kv_dim];
        let mut v = vec![0f32; n * self.kv_dim];
        check(unsafe { ltkv_rows(self.raw, layer, seq, n, k.as_mut_ptr().cast(), v.as_mut_ptr().cast()) })?;
        Ok((k, v))
    }

    /// kv.rs:153-169 (`Backend::kv_remove`).
    pub fn truncate(&mut self, seq: u32, from: usize) {
        unsafe { ltkv_truncate(self.raw, seq, from) }
    }

    /// kv.rs:172-183 (`Backend::kv_copy`).
    pub fn share(&mut self, src: u32, dst: u32, len: usize) {
        unsafe { ltkv_share(self.raw, src, dst, len) }
    }

    /// The block table of `seq` (Seq::blocks, kv.rs:28-32).
    pub fn block_table(&self, seq: u32) -> anyhow::Result<Vec<i32>> {
        let mut n = 0usize;
        check(unsafe { ltkv_block_table(self.raw, seq, std::ptr::null_mut(), 0, &mut n) }).or_else(|e| {
            if n > 0 { Ok(()) } else { Err(e) }
        })?;
        let mut out = vec![0i32; n];
        check(unsafe { ltkv_block_table(self.raw, seq, out.as_mut_ptr(), n, &mut n) })?;
        Ok(out)
    }

    /// Row-major [seqs.len()][stride] tables, -1 past each table's end.
    pub fn block_tables(&self, seqs: &[u32], stride: usize) -> anyhow::Result<Vec<i32>> {
        let mut out = vec![0i32; seqs.len() * stride];
        check(unsafe { ltkv_block_tables(self.raw, seqs.len(), seqs.as_ptr(), out.as_mut_ptr(), stride) })?;
        Ok(out)
    }

    pub fn init_free_order(&mut self, order: &[u32]) -> anyhow::Result<()> {
        check(unsafe { ltkv_init_free_order(self.raw, order.as_ptr(), order.len()) })
    }

    pub fn set_attention_partition(&mut self, tokens: usize) -> anyhow::Result<()> {
        check(unsafe { ltkv_set_attention_partition(self.raw, tokens) })
    }

    /// `LTKV_ENGINE_AUTO` or `LTKV_ENGINE_VALU` (f16 pools on the vector ALU).
    pub fn set_attention_engine(&mut self, engine: c_int) -> anyhow::Result<()> {
        check(unsafe { ltkv_set_attention_engine(self.raw, engine) })
    }

    pub fn rope_init(&mut self, base: f32, rope_dim: usize, head_dim: usize, neox: bool,
                     max_positions: usize) -> anyhow::Result<()> {
        check(unsafe { ltkv_rope_init(self.raw, base, rope_dim, head_dim, neox as c_int, max_positions) })
    }

    /// Plans one batch's attention (every layer of the step reuses it).
    /// `f16_products`: grouped products on f16-rounded Q and weights (faster,
    /// ~3e-4 relative error instead of f32 accuracy).
    pub fn plan_attention(&mut self, seqs: &[u32], lens: &[u32], n_heads: usize, head_dim: usize,
                          shared_prefix: bool, f16_products: bool) -> anyhow::Result<()> {
        anyhow::ensure!(seqs.len() == lens.len(), "seqs and lens differ in length");
        let flags = (if shared_prefix { LTKV_PLAN_SHARED_PREFIX } else { 0 })
            | (if f16_products { LTKV_PLAN_F16_PRODUCTS } else { 0 });
        check(unsafe { ltkv_plan_attention(self.raw, seqs.len(), seqs.as_ptr(), lens.as_ptr(), n_heads, head_dim, flags) })
    }

    pub fn plan_stats(&self) -> anyhow::Result<[u64; 6]> {
        let mut out = [0u64; 6];
        check(unsafe { ltkv_plan_stats(self.raw, out.as_mut_ptr()) })?;
        Ok(out)
    }

    pub fn seq_rows(&self, seqs: &[u32]) -> anyhow::Result<Vec<i32>> {
        let mut rows = vec![0i32; seqs.len()];
        check(unsafe { ltkv_seq_rows(self.raw, seqs.len(), seqs.as_ptr(), rows.as_mut_ptr()) })?;
        Ok(rows)
    }

    pub fn sync_tables(&mut self) -> anyhow::Result<()> {
        check(unsafe { ltkv_sync_tables(self.raw) })
    }

    /// (device tables, device lengths, stride, rows) of the resident tables.
    pub fn resident_tables(&mut self) -> anyhow::Result<(*const i32, *const i32, usize, usize)> {
        let (mut t, mut l) = (std::ptr::null(), std::ptr::null());
        let (mut stride, mut rows) = (0usize, 0usize);
        check(unsafe { ltkv_resident_tables(self.raw, &mut t, &mut l, &mut stride, &mut rows) })?;
        Ok((t, l, stride, rows))
    }

    /// The resident tables on the host: `tables` takes stride * rows entries
    /// and `lengths` rows entries, as `resident_tables` reports them.
    pub fn read_resident_tables(&mut self, tables: &mut [i32], lengths: &mut [i32]) -> anyhow::Result<()> {
        let (_, _, stride, rows) = self.resident_tables()?;
        anyhow::ensure!(tables.len() >= stride * rows && lengths.len() >= rows,
                        "buffers hold {} table entries and {} lengths; the tables need {} and {}",
                        tables.len(), lengths.len(), stride * rows, rows);
        check(unsafe { ltkv_read_resident_tables(self.raw, tables.as_mut_ptr(), lengths.as_mut_ptr()) })
    }

    pub fn table_uploads(&self) -> anyhow::Result<u64> {
        let mut n = 0u64;
        check(unsafe { ltkv_table_uploads(self.raw, &mut n) })?;
        Ok(n)
    }

    /// One layer's K and V pools to host ([n_blocks][16][kv_dim] elements of
    /// the cache's dtype: f16 bits, f32, or Q8_0 quants).
    pub unsafe fn read_pool(&mut self, layer: usize, h_k: *mut c_void, h_v: *mut c_void) -> anyhow::Result<()> {
        check(ltkv_read_pool(self.raw, layer, h_k, h_v))
    }

    /// One layer's K and V scale pools of a Q8_0 cache: n_blocks * (kv_dim / 32)
    /// * 16 f16 bits each, [block][group][slot].
    pub fn read_scales(&mut self, layer: usize, h_k: &mut [u16], h_v: &mut [u16]) -> anyhow::Result<()> {
        let need = self.n_blocks() * (self.kv_dim / 32) * 16;
        anyhow::ensure!(h_k.len() >= need && h_v.len() >= need,
                        "scale buffers hold {} and {} entries; a layer has {}", h_k.len(), h_v.len(), need);
        check(unsafe { ltkv_read_scales(self.raw, layer, h_k.as_mut_ptr(), h_v.as_mut_ptr()) })
    }

    pub fn synchronize(&mut self) -> anyhow::Result<()> {
        check(unsafe { ltkv_synchronize(self.raw) })
    }

    // ---- device ops: raw device pointers, enqueued on the cache's stream

    /// Kernel 1 (kv.rs:123-131 for n rows, model.rs:414-429).
    pub unsafe fn write_device(&mut self, layer: usize, n: usize, d_slot_mapping: *const i32, d_k: *const f32,
                               d_v: *const f32, src_stride: usize) -> anyhow::Result<()> {
        check(ltkv_write(self.raw, layer, n, d_slot_mapping, d_k, d_v, src_stride))
    }

    /// The rows of a claimed batch grouped by block in ascending block order
    /// (host only), for `write_ordered`.
    pub fn cell_order(&self, slot_mapping: &[i32]) -> anyhow::Result<Vec<i32>> {
        let mut order = vec![0i32; slot_mapping.len()];
        let mut m = 0usize;
        check(unsafe {
            ltkv_cell_order(self.raw, slot_mapping.len(), slot_mapping.as_ptr(), order.as_mut_ptr(), &mut m)
        })?;
        order.truncate(m);
        Ok(order)
    }

    /// Kernel 1 over the rows `d_order[0..m)` of a batch of `n` rows.
    pub unsafe fn write_ordered(&mut self, layer: usize, n: usize, d_slot_mapping: *const i32, d_k: *const f32,
                                d_v: *const f32, src_stride: usize, m: usize,
                                d_order: *const i32) -> anyhow::Result<()> {
        check(ltkv_write_ordered(self.raw, layer, n, d_slot_mapping, d_k, d_v, src_stride, m, d_order))
    }

    /// RoPE (model.rs:291-308) fused into kernel 1; Q rotated in place.
    pub unsafe fn write_rope(&mut self, layer: usize, n: usize, d_slot_mapping: *const i32, d_positions: *const i32,
                             d_k: *const f32, d_v: *const f32, src_stride: usize, d_q: *mut f32, q_stride: usize,
                             n_heads: usize) -> anyhow::Result<()> {
        check(ltkv_write_rope(self.raw, layer, n, d_slot_mapping, d_positions, d_k, d_v, src_stride, d_q, q_stride,
                              n_heads))
    }

    /// Kernel 2 (the copy-on-write body of kv.rs:99-110) for device (src, dst) pairs.
    pub unsafe fn copy_blocks(&mut self, n: usize, d_pairs: *const i32) -> anyhow::Result<()> {
        check(ltkv_copy_blocks(self.raw, n, d_pairs))
    }

    /// Kernel 3 (kv.rs:133-150 collected) for n sequences.
    pub unsafe fn gather(&mut self, layer: usize, n: usize, d_tables: *const i32, table_stride: usize,
                         d_lens: *const i32, d_out_offsets: *const i64, d_k_out: *mut c_void,
                         d_v_out: *mut c_void) -> anyhow::Result<()> {
        check(ltkv_gather(self.raw, layer, n, d_tables, table_stride, d_lens, d_out_offsets, d_k_out, d_v_out))
    }

    /// Kernel 4 (the attention closure of model.rs:431-475).
    pub unsafe fn decode_attention(&mut self, layer: usize, n: usize, n_heads: usize, head_dim: usize, scale: f32,
                                   d_q: *const f32, d_tables: *const i32, table_stride: usize, d_lens: *const i32,
                                   d_out: *mut f32) -> anyhow::Result<()> {
        check(ltkv_decode_attention(self.raw, layer, n, n_heads, head_dim, scale, d_q, d_tables, table_stride, d_lens,
                                    d_out))
    }

    /// Kernel 4 with nothing allocated (partials in the device's static scratch).
    pub unsafe fn decode_attention_noalloc(&mut self, layer: usize, n: usize, n_heads: usize, head_dim: usize,
                                           scale: f32, d_q: *const f32, d_tables: *const i32, table_stride: usize,
                                           d_lens: *const i32, d_out: *mut f32) -> anyhow::Result<()> {
        check(ltkv_decode_attention_noalloc(self.raw, layer, n, n_heads, head_dim, scale, d_q, d_tables,
                                            table_stride, d_lens, d_out))
    }

    /// A decode step's append and attention in one launch (model.rs:414-475).
    pub unsafe fn append_decode_attention(&mut self, layer: usize, n: usize, n_heads: usize, head_dim: usize,
                                          scale: f32, d_q: *const f32, d_tables: *const i32, table_stride: usize,
                                          d_lens: *const i32, d_slot_mapping: *const i32, d_k: *const f32,
                                          d_v: *const f32, src_stride: usize, d_out: *mut f32) -> anyhow::Result<()> {
        check(ltkv_append_decode_attention(self.raw, layer, n, n_heads, head_dim, scale, d_q, d_tables, table_stride,
                                           d_lens, d_slot_mapping, d_k, d_v, src_stride, d_out))
    }

    pub unsafe fn planned_attention(&mut self, layer: usize, scale: f32, d_q: *const f32,
                                    d_out: *mut f32) -> anyhow::Result<()> {
        check(ltkv_planned_attention(self.raw, layer, scale, d_q, d_out))
    }

    pub unsafe fn slot_mapping(&mut self, n: usize, d_rows: *const i32, d_pos: *const i64,
                               d_slot_mapping: *mut i32) -> anyhow::Result<()> {
        check(ltkv_slot_mapping(self.raw, n, d_rows, d_pos, d_slot_mapping))
    }

    pub unsafe fn decode_attention_rows(&mut self, layer: usize, n: usize, n_heads: usize, head_dim: usize,
                                        scale: f32, d_q: *const f32, d_rows: *const i32, d_lens: *const i32,
                                        d_out: *mut f32) -> anyhow::Result<()> {
        check(ltkv_decode_attention_rows(self.raw, layer, n, n_heads, head_dim, scale, d_q, d_rows, d_lens, d_out))
    }
}
