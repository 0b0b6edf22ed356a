"""Block copy, swap and kv_exchange pack/scatter on the GPU: bit-exact."""
import numpy as np
import pytest
import torch

import kunserve_amd
from kunserve_amd import KVPool, LlamaOp, copy_blocks, kv_pack, kv_scatter, swap, workloads
from oracle import paged_attention_ref as ref

pytestmark = pytest.mark.gpu


def unique_pool(shape, device, offset=0, chunk_pages=512):
    """Pool whose int16 bit patterns encode the element index, viewed as fp16
    (bit-exact comparisons only; nothing computes on these values). Filled
    in page chunks to bound the temporary index tensor."""
    out = torch.empty(shape, dtype=torch.int16, device=device)
    per_page = int(np.prod(shape[1:]))
    for p0 in range(0, shape[0], chunk_pages):
        p1 = min(shape[0], p0 + chunk_pages)
        idx = torch.arange(p0 * per_page, p1 * per_page, device=device, dtype=torch.int64)
        out[p0:p1].view(-1).copy_(((idx * 7 + offset) % 65536).to(torch.int32).to(torch.int16))
    return out.view(torch.float16)


def test_copy_blocks_matches_oracle(device):
    shape = (64, 3, 2, 16, 128)
    pool = KVPool(unique_pool(shape, device), unique_pool(shape, device, 1))
    k0, v0 = pool.k.view(torch.int16).cpu().numpy(), pool.v.view(torch.int16).cpu().numpy()
    rng = np.random.default_rng(0)
    ids = rng.permutation(64)
    src, dst = ids[:20].tolist(), ids[20:40].tolist()
    copy_blocks(pool, src, dst)
    torch.cuda.synchronize()
    ref.copy_blocks(k0, src, dst)
    ref.copy_blocks(v0, src, dst)
    assert np.array_equal(pool.k.view(torch.int16).cpu().numpy(), k0)
    assert np.array_equal(pool.v.view(torch.int16).cpu().numpy(), v0)


def test_copy_blocks_layer_major_pool(device):
    """A pool whose pages are not contiguous (layer-major storage viewed as
    [pages, layers, ...]) is copied per layer slab."""
    L, P = 4, 32
    store_k = unique_pool((L, P, 2, 16, 64), device)
    store_v = unique_pool((L, P, 2, 16, 64), device, 3)
    pool = KVPool(store_k.transpose(0, 1), store_v.transpose(0, 1))
    k0 = pool.k.contiguous().view(torch.int16).cpu().numpy()
    src, dst = [1, 2, 30], [5, 0, 31]
    copy_blocks(pool, src, dst)
    torch.cuda.synchronize()
    ref.copy_blocks(k0, src, dst)
    assert np.array_equal(pool.k.contiguous().view(torch.int16).cpu().numpy(), k0)


def test_copy_rejects_bad_ids(device):
    pool = KVPool.allocate(8, 1, 1, 16, 64, device)
    with pytest.raises(IndexError):
        copy_blocks(pool, [0, 8], [1, 2])
    op = LlamaOp(8, 1, 1, 1, 16, 64, 1, 1, 1, 1, 1, 1, device)
    with pytest.raises(ValueError):
        op.local_copy_blocks(8, [1, 2], [2, 3])   # overlapping src/dst


def test_remap_copy_8192_blocks_bit_exact(device):
    """8192 random 2 MiB blocks (32 layers x 8 heads x 16 x 128, K and V)
    between disjoint regions: every destination equals its source."""
    r = workloads.kv_remap()
    n_pages = 2 * len(r.src)
    shape = (n_pages, r.num_layers, r.num_kv_heads, r.page_size, r.head_dim)
    pool = KVPool(unique_pool(shape, device), unique_pool(shape, device, 5))
    copy_blocks(pool, r.src, r.dst)
    torch.cuda.synchronize()
    s = torch.from_numpy(r.src.astype(np.int64)).to(device)
    d = torch.from_numpy(r.dst.astype(np.int64)).to(device)
    n = len(r.src)
    for t, off in ((pool.k, 0), (pool.v, 5)):
        for c in range(0, n, 1024):
            sc, dc = s[c:c + 1024], d[c:c + 1024]
            assert torch.equal(t.index_select(0, dc).view(torch.int16),
                               t.index_select(0, sc).view(torch.int16))
        # the source region is untouched
        fresh = unique_pool(shape, device, off)
        assert torch.equal(t[:n].view(torch.int16), fresh[:n].view(torch.int16))
        del fresh


def test_swap_out_and_in_round_trip(device):
    shape = (16, 2, 4, 16, 128)
    k = unique_pool(shape, device)
    v = unique_pool(shape, device, 9)
    ks = torch.zeros((10,) + shape[1:], dtype=torch.float16, pin_memory=True)
    vs = torch.zeros((10,) + shape[1:], dtype=torch.float16, pin_memory=True)
    src, dst = [3, 4, 5, 9, 0], [0, 1, 2, 7, 9]   # one merged run of three
    torch.ops.swapping_ops.swap(src, dst, False, k, v, ks, vs)
    torch.cuda.synchronize()
    kn = k.view(torch.int16).cpu().numpy()
    host = np.zeros((10,) + shape[1:], dtype=np.int16)
    ref.swap(src, dst, kn, host)
    assert np.array_equal(ks.view(torch.int16).numpy(), host)
    # swap back into different GPU blocks
    k2, v2 = torch.zeros_like(k), torch.zeros_like(v)
    swap([0, 7], [11, 12], True, k2, v2, ks, vs)
    torch.cuda.synchronize()
    assert torch.equal(k2[11].view(torch.int16), k[3].view(torch.int16))
    assert torch.equal(v2[12].view(torch.int16), v[9].view(torch.int16))
    assert not k2[:11].view(torch.int16).any()


def test_swap_through_the_abi_with_pageable_host_pools(device):
    """Host pools the device cannot map (plain pageable memory) take the
    fallback: one DMA copy per run of consecutive ids, both directions."""
    import ctypes
    from kunserve_amd import _lib
    shape = (12, 2, 2, 16, 64)
    k = unique_pool(shape, device)
    v = unique_pool(shape, device, 5)
    block_bytes = int(np.prod(shape[1:])) * 2
    kh = np.zeros((8,) + shape[1:], dtype=np.int16)
    vh = np.zeros((8,) + shape[1:], dtype=np.int16)
    stream = torch.cuda.current_stream(device).cuda_stream

    def call(src, dst, is_in, n_dev, n_host):
        s = np.asarray(src, dtype=np.int64)
        d = np.asarray(dst, dtype=np.int64)
        _lib.call("kunserve_swap_blocks", s.ctypes.data, d.ctypes.data, len(s), int(is_in),
                  k.data_ptr(), v.data_ptr(), n_dev, kh.ctypes.data, vh.ctypes.data, n_host,
                  block_bytes, stream)
        torch.cuda.synchronize()

    src, dst = [3, 4, 5, 9, 0], [0, 1, 2, 6, 7]   # a run of three, then two singles
    call(src, dst, False, 12, 8)
    want_k = np.zeros_like(kh)
    want_v = np.zeros_like(vh)
    ref.swap(src, dst, k.view(torch.int16).cpu().numpy(), want_k)
    ref.swap(src, dst, v.view(torch.int16).cpu().numpy(), want_v)
    assert np.array_equal(kh, want_k) and np.array_equal(vh, want_v)
    k_before = k.view(torch.int16).cpu().numpy()
    call([0, 1, 2, 7], [10, 11, 8, 4], True, 12, 8)
    want = k_before.copy()
    ref.swap([0, 1, 2, 7], [10, 11, 8, 4], kh, want)
    assert np.array_equal(k.view(torch.int16).cpu().numpy(), want)
    with pytest.raises(_lib.KunserveError):
        call([8], [0], True, 12, 8)   # host block 8 is outside [0, 8)


def test_swap_on_side_stream_is_ordered(device):
    shape = (4, 1, 2, 16, 64)
    k = unique_pool(shape, device)
    v = unique_pool(shape, device, 2)
    ks = torch.zeros(shape, dtype=torch.float16, pin_memory=True)
    vs = torch.zeros(shape, dtype=torch.float16, pin_memory=True)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        torch.ops.swapping_ops.swap([1], [2], False, k, v, ks, vs)
        ev = torch.cuda.Event()
        ev.record(stream)
    ev.synchronize()
    assert torch.equal(ks[2].view(torch.int16), k[1].view(torch.int16).cpu())


def test_swap_views_into_larger_pinned_tensors(device):
    """Host pools that start inside a larger pinned allocation (the caching
    host allocator hands out such views)."""
    shape = (6, 2, 2, 16, 128)
    k = unique_pool(shape, device)
    v = unique_pool(shape, device, 5)
    big_k = torch.zeros((9,) + shape[1:], dtype=torch.float16, pin_memory=True)
    big_v = torch.zeros((9,) + shape[1:], dtype=torch.float16, pin_memory=True)
    ks, vs = big_k[3:8], big_v[2:7]
    swap([5, 0, 2], [4, 0, 1], False, k, v, ks, vs)
    torch.cuda.synchronize()
    for s_, d in zip([5, 0, 2], [4, 0, 1]):
        assert torch.equal(ks[d].view(torch.int16), k[s_].view(torch.int16).cpu())
        assert torch.equal(vs[d].view(torch.int16), v[s_].view(torch.int16).cpu())
    # nothing outside the views was written
    assert not big_k[:3].view(torch.int16).any() and not big_k[8:].view(torch.int16).any()
    assert not big_v[:2].view(torch.int16).any() and not big_v[7:].view(torch.int16).any()


def test_many_swaps_in_flight_without_sync(device):
    """Back-to-back swaps on one stream with no host wait between them: each
    call's id lists must stay intact until its copies ran, and stream order
    must hold (the same GPU block goes out, is overwritten, goes out again)."""
    shape = (8, 1, 2, 16, 64)
    k = unique_pool(shape, device)
    v = unique_pool(shape, device, 3)
    n_calls = 150   # more than the id slots kept per device
    ks = torch.zeros((n_calls,) + shape[1:], dtype=torch.float16, pin_memory=True)
    vs = torch.zeros((n_calls,) + shape[1:], dtype=torch.float16, pin_memory=True)
    want_k = []
    for c in range(n_calls):
        src = c % shape[0]
        k.view(torch.int16)[src].add_(1)   # changes the block between swaps, in stream order
        want_k.append(k[src].clone())
        swap([src], [c], False, k, v, ks, vs)
    torch.cuda.synchronize()
    for c in range(n_calls):
        assert torch.equal(ks[c].view(torch.int16), want_k[c].view(torch.int16).cpu()), c
        assert torch.equal(vs[c].view(torch.int16), v[c % shape[0]].view(torch.int16).cpu()), c


def test_pack_scatter_round_trip(device):
    shape = (40, 6, 2, 16, 128)
    a = KVPool(unique_pool(shape, device), unique_pool(shape, device, 4))
    ids = [7, 3, 22, 39]
    scr = kv_pack(a, 2, 5, ids)
    torch.cuda.synchronize()
    want = ref.kv_pack(a.k.view(torch.int16).cpu().numpy(), a.v.view(torch.int16).cpu().numpy(),
                       2, 5, ids)
    got = scr.view(torch.int16).cpu().numpy()[:want.size].reshape(want.shape)
    assert np.array_equal(got, want)
    b = KVPool(torch.zeros_like(a.k), torch.zeros_like(a.v))
    dst = [0, 10, 11, 30]
    kv_scatter(b, 2, 5, dst, scr)
    torch.cuda.synchronize()
    for s, d in zip(ids, dst):
        assert torch.equal(b.k[d, 2:5].view(torch.int16), a.k[s, 2:5].view(torch.int16))
        assert torch.equal(b.v[d, 2:5].view(torch.int16), a.v[s, 2:5].view(torch.int16))
    assert not b.k[:, :2].view(torch.int16).any() and not b.k[:, 5:].view(torch.int16).any()


def test_llama_op_exchange_loopback(device):
    """Two LlamaOps on one GPU: instance A packs its stale pages, instance B
    (stage 1 of a 2-instance group) scatters them into its fused ids — the
    single-GPU halves of kv_exchange. Fused id 1*P + b is layers [2, 4) of
    B's page b (the oracle's fused map)."""
    a = LlamaOp(32, 4, 4, 2, 16, 128, 1, 1, 1, 1, 1, 1, device)
    b = LlamaOp(32, 4, 4, 2, 16, 128, 1, 1, 1, 1, 1, 1, device)
    a.pool.k.copy_(unique_pool(a.pool.k.shape, device))
    a.pool.v.copy_(unique_pool(a.pool.v.shape, device, 8))
    b.pool.k.zero_()
    b.pool.v.zero_()
    b.pmm_drop(1, 2)
    src = sorted([9, 2, 13])          # pre-fusion ids < P = 32
    fused = [ref.kept_page_id(p, 64, 2, 1) for p in (20, 5, 31)]
    scr = a.kv_exchange_pack(src, 2, 4)
    b.kv_exchange_scatter(fused, 2, 4, scr)
    torch.cuda.synchronize()
    bk = ref.fused_pool_copy(b.pool.k.cpu().numpy(), 32, 2)
    bv = ref.fused_pool_copy(b.pool.v.cpu().numpy(), 32, 2)
    for s, d in zip(src, fused):
        assert np.array_equal(bk[d].view(np.int16), a.pool.k[s, 2:4].cpu().numpy().view(np.int16))
        assert np.array_equal(bv[d].view(np.int16), a.pool.v[s, 2:4].cpu().numpy().view(np.int16))
    for page, layer in [(20, 0), (20, 1), (5, 0), (31, 1)]:   # the other layer group is untouched
        assert not b.pool.k[page, layer].view(torch.int16).any()
    a.kv_exchange([[1], [2]], 0, 1, 0, 1, 32, 0)      # group of one: no-op
    with pytest.raises(NotImplementedError):
        a.kv_exchange([[1], [2]], 0, 1, 0, 2, 32, 0)
