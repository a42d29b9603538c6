"""ltkv_decode_attention_noalloc: decode attention whose partition partials
live in the device's static scratch instead of a workspace allocated on
demand. It runs the same kernels as ltkv_decode_attention, so its outputs
must equal that entry point's bit for bit: checked on two calls in a row
(the second with a smaller batch, so it overwrites part of what the first
left in the scratch), on a fresh cache whose first attention call is the
no-allocation one, for f16, q8_0 (partitions cut in two) and f32 pools. A
launch whose partials exceed the scratch is refused before anything runs; a
call leaves the device's free memory unchanged; shapes outside the tuned
kernels (no partials) are taken at any table stride."""

from __future__ import annotations

import numpy as np
import pytest

from helpers import BLOCK

pytestmark = pytest.mark.gpu


def _filled(dtype, n_kv, hd, ctx, seed):
    import torch

    from langtrain_studio_amd import KvCache

    kvd = n_kv * hd
    rng = np.random.default_rng(seed)
    n_blocks = int(sum(-(-int(c) // BLOCK) for c in ctx) * 1.1) + 8
    kv = KvCache(1, kvd, n_blocks * BLOCK, dtype=dtype, device=0, stream=torch.cuda.current_stream())
    kv.init_free_order(rng.permutation(n_blocks))
    seqs = np.repeat(np.arange(len(ctx), dtype=np.uint32), ctx)
    pos = np.concatenate([np.arange(int(c), dtype=np.uint64) for c in ctx])
    sm = kv.append_batch(seqs, pos)
    gen = torch.Generator(device="cuda").manual_seed(seed)
    k = torch.randn((sm.size, kvd), generator=gen, device="cuda")
    v = torch.randn((sm.size, kvd), generator=gen, device="cuda")
    kv.write_batch(0, torch.from_numpy(sm).cuda(), k, v)
    return kv


@pytest.mark.parametrize("dtype,n_heads,n_kv,hd,lo,hi", [
    ("f16", 32, 8, 128, 2048, 4097),   # Llama-3-8B decode shape, two kv heads per wave
    ("q8_0", 32, 8, 128, 3000, 9000),  # partitions cut in two; some queries beyond 4096 tokens
    ("f16", 28, 4, 128, 512, 8193),    # Qwen2.5-7B, one kv head per wave, up to 9 partitions
    ("f16", 32, 8, 128, 11000, 13001),  # over twice the wave slots in partitions: runs per wave
    ("f32", 32, 4, 64, 128, 513),      # TinyLlama shape, vector-ALU kernel
])
def test_noalloc_equals_decode_attention(gpu, dtype, n_heads, n_kv, hd, lo, hi):
    import torch

    rng = np.random.default_rng(hi + n_heads)
    B = 48
    ctx = rng.integers(lo, hi, B)
    print(f"noalloc {dtype} {n_heads}/{n_kv}/{hd} B={B} ctx [{lo},{hi})", flush=True)
    kv = _filled(dtype, n_kv, hd, ctx, int(hi))
    tables = torch.from_numpy(kv.block_tables(np.arange(B, dtype=np.uint32))).cuda()
    lens = torch.from_numpy(ctx.astype(np.int32)).cuda()
    q = torch.randn((B, n_heads * hd), generator=torch.Generator(device="cuda").manual_seed(7), device="cuda")
    small = np.array([3, 11, 30])
    q_s, t_s, l_s = (q[small].contiguous(), tables[small, : (tables.shape[1] + 1) // 2].contiguous(),
                     lens[small] // 2)

    # two calls in a row on the no-allocation entry point, the second smaller
    big_na = kv.decode_attention(0, q, tables, lens, n_heads, hd, noalloc=True).cpu().numpy()
    small_na = kv.decode_attention(0, q_s, t_s, l_s, n_heads, hd, noalloc=True).cpu().numpy()
    # the allocating entry point on the same inputs
    big = kv.decode_attention(0, q, tables, lens, n_heads, hd).cpu().numpy()
    small_ref = kv.decode_attention(0, q_s, t_s, l_s, n_heads, hd).cpu().numpy()
    assert np.isfinite(big).all() and np.abs(big).max() > 0
    np.testing.assert_array_equal(big_na.view(np.uint32), big.view(np.uint32))
    np.testing.assert_array_equal(small_na.view(np.uint32), small_ref.view(np.uint32))
    # and once more after the allocating calls used the cache's own workspace
    again = kv.decode_attention(0, q_s, t_s, l_s, n_heads, hd, noalloc=True).cpu().numpy()
    np.testing.assert_array_equal(again.view(np.uint32), small_ref.view(np.uint32))


def test_noalloc_refuses_partials_beyond_the_scratch(gpu):
    """64 queries over tables of 4096 blocks (65 536 tokens: 64 partitions of
    1024) need 64 x 32 x 64 x 130 x 4 B = 68 MB of partials, more than the
    32 MiB scratch: refused on the host with LTKV_ERR_ARG, no launch."""
    import torch

    from langtrain_studio_amd import KvError, _lib

    kv = _filled("f16", 8, 128, np.full(4, 64), 1)
    B, stride = 64, 4096
    tables = torch.full((B, stride), -1, dtype=torch.int32, device="cuda")
    lens = torch.zeros(B, dtype=torch.int32, device="cuda")
    q = torch.zeros((B, 32 * 128), device="cuda")
    need = B * 32 * (stride * BLOCK // 1024) * (128 + 2) * 4
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    with pytest.raises(KvError, match="no-allocation scratch") as e:
        kv.decode_attention(0, q, tables, lens, 32, 128, noalloc=True)
    assert e.value.code == _lib.ERR_ARG
    # the allocating entry point takes the same launch (all lengths 0: zeros)
    out = kv.decode_attention(0, q, tables, lens, 32, 128)
    assert not out.any()


def test_noalloc_allocates_nothing(gpu):
    """A fresh cache's first attention call through the no-allocation entry
    point leaves the device's free memory as it was; the allocating entry
    point on the same launch then grows the cache's workspace by the ~30 MB
    of partials (64 queries x 32 heads x 28 partitions x 130 floats), so the
    measurement sees such a growth."""
    import torch

    B, stride = 64, 1792  # tables of 28 672 tokens: 28 partitions of 1024
    ctx = np.random.default_rng(5).integers(100, 3000, B)
    kv = _filled("f16", 8, 128, ctx, 5)
    tables = torch.full((B, stride), -1, dtype=torch.int32, device="cuda")
    t = torch.from_numpy(kv.block_tables(np.arange(B, dtype=np.uint32))).cuda()
    tables[:, :t.shape[1]] = t
    lens = torch.from_numpy(ctx.astype(np.int32)).cuda()
    q = torch.randn((B, 32 * 128), generator=torch.Generator(device="cuda").manual_seed(9), device="cuda")
    out_na, out = torch.empty_like(q), torch.empty_like(q)
    # the same launch once on another cache first, so that whatever the
    # runtime sets up at a kernel's first launch is not counted
    warm = _filled("f16", 8, 128, ctx[:4], 5)
    w_tables = torch.full((4, stride), -1, dtype=torch.int32, device="cuda")
    wt = torch.from_numpy(warm.block_tables(np.arange(4, dtype=np.uint32))).cuda()
    w_tables[:, :wt.shape[1]] = wt
    warm.decode_attention(0, q[:4].contiguous(), w_tables, lens[:4].contiguous(), 32, 128, noalloc=True)
    warm.synchronize()
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    kv.decode_attention(0, q, tables, lens, 32, 128, out=out_na, noalloc=True)
    kv.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0, f"the no-allocation call changed free device memory by {free0 - free1} bytes"
    kv.decode_attention(0, q, tables, lens, 32, 128, out=out)
    kv.synchronize()
    free2, _ = torch.cuda.mem_get_info()
    assert free1 - free2 >= 16 << 20, "the workspace growth is not visible in the free-memory figure"
    assert torch.equal(out_na.view(torch.int32), out.view(torch.int32))


def test_noalloc_generic_shape_takes_any_table_stride(gpu):
    """Shapes outside the tuned kernels (here head_dim 96 with 16 query heads
    a kv head) run the generic kernel over whole contexts and write no
    partials, so the no-allocation entry point takes them whatever the table
    stride (4096 blocks: 64 partitions would need 51 MB of partials), with
    the allocating entry point's bits."""
    import torch

    B, stride, n_heads, n_kv, hd = 64, 4096, 32, 2, 96
    ctx = np.random.default_rng(6).integers(1, 700, B)
    kv = _filled("f16", n_kv, hd, ctx, 6)
    tables = torch.full((B, stride), -1, dtype=torch.int32, device="cuda")
    t = torch.from_numpy(kv.block_tables(np.arange(B, dtype=np.uint32))).cuda()
    tables[:, :t.shape[1]] = t
    lens = torch.from_numpy(ctx.astype(np.int32)).cuda()
    q = torch.randn((B, n_heads * hd), generator=torch.Generator(device="cuda").manual_seed(10), device="cuda")
    na = kv.decode_attention(0, q, tables, lens, n_heads, hd, noalloc=True).cpu().numpy()
    ref = kv.decode_attention(0, q, tables, lens, n_heads, hd).cpu().numpy()
    assert np.isfinite(na).all() and np.abs(na).max() > 0
    np.testing.assert_array_equal(na.view(np.uint32), ref.view(np.uint32))
