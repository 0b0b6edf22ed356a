"""The calibration probes the benchmark uses for its ceilings, checked against
closed forms: the MFMA probe's per-wave sums, and the HBM probe's copy mode."""
import numpy as np
import pytest
import torch

from kunserve_amd import _lib

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype_code,dtype", [(0, torch.float16), (1, torch.bfloat16)])
def test_mfma_probe_matches_closed_form(dtype_code, dtype):
    """Lane l of a wave holds row / column l % 32 and k-block l // 32 of both
    32x32x16 operands, so the sum of every accumulator entry of x.y (and of
    y.x) is sum over (k-block h, element e) of X[h, e] * Y[h, e], with X and Y
    the operands summed over the 32 lanes of block h. Small integers keep
    every sum exact in fp32."""
    dev = torch.device("cuda", 0)
    wg, iters = 3, 5
    rng = np.random.default_rng(11)
    ops = rng.integers(-4, 5, size=wg * 512 * 16)
    sink = torch.full((wg * 512,), float("nan"), dtype=torch.float32, device=dev)
    ops_dev = torch.from_numpy(ops.astype(np.float32)).to(dtype).to(dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    _lib.call("kunserve_mfma_probe", dtype_code, ops_dev.data_ptr(), sink.data_ptr(), wg, iters,
              stream)
    torch.cuda.synchronize()
    per_lane = ops.reshape(wg * 8, 2, 32, 16)       # wave, k-block, lane in block, x | y
    xs = per_lane[..., :8].sum(axis=2)             # [wave, k-block, e]
    ys = per_lane[..., 8:].sum(axis=2)
    want = iters * 2 * (xs * ys).sum(axis=(1, 2))
    got = sink.view(wg * 8, 64).sum(dim=1, dtype=torch.float64).cpu().numpy()
    np.testing.assert_array_equal(got, want)


def test_mfma_probe_rejects_bad_arguments():
    dev = torch.device("cuda", 0)
    ops = torch.zeros(512 * 16, dtype=torch.float16, device=dev)
    sink = torch.empty(512, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    with pytest.raises(_lib.KunserveError):
        _lib.call("kunserve_mfma_probe", 2, ops.data_ptr(), sink.data_ptr(), 1, 1, stream)
    with pytest.raises(_lib.KunserveError):
        _lib.call("kunserve_mfma_probe", 0, ops.data_ptr(), sink.data_ptr(), 0, 1, stream)
    with pytest.raises(_lib.KunserveError):
        _lib.call("kunserve_mfma_probe", 0, None, sink.data_ptr(), 1, 1, stream)


def test_hbm_probe_copy_is_exact():
    """Mode 2 copies the bytes; mode 1 overwrites the destination."""
    dev = torch.device("cuda", 0)
    chunk = 256 * 1024
    src = torch.randint(0, 256, (4 * chunk,), dtype=torch.uint8, device=dev)
    dst = torch.zeros_like(src)
    stream = torch.cuda.current_stream(dev).cuda_stream
    _lib.call("kunserve_hbm_probe", 2, src.data_ptr(), dst.data_ptr(), src.numel(), stream)
    torch.cuda.synchronize()
    assert torch.equal(src, dst)
    _lib.call("kunserve_hbm_probe", 1, None, dst.data_ptr(), dst.numel(), stream)
    torch.cuda.synchronize()
    assert not torch.equal(src, dst)


@pytest.mark.parametrize("page_size,head_dim", [(16, 128), (16, 64), (64, 128)])
def test_decode_slab_probe_reads_the_slabs(page_size, head_dim):
    """The slab probe XORs exactly the words of its items' slabs (K and V,
    every head) into one word per workgroup, reading a count above
    max_slabs as max_slabs; bad arguments are rejected."""
    from kunserve_amd import KVPool
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev)
    g.manual_seed(page_size + head_dim)
    pool = KVPool.allocate(40, 2, 3, page_size, head_dim, dev)
    for t in (pool.k, pool.v):
        t.copy_(torch.randn(t.shape, generator=g, device=dev))
    rng = np.random.default_rng(0)
    counts = np.array([5, 0, 1, 11, 2, 0, 0, 3], dtype=np.int32)   # 8 items: one per XCD lane
    max_slabs = 8
    layer = 1
    es = pool.k.element_size()
    pages = np.zeros((8, max_slabs), dtype=np.int64)
    used = np.minimum(counts, max_slabs)
    for i, n in enumerate(used):
        pages[i, :n] = rng.choice(40, size=n, replace=False)
    offs = pages * pool.k.stride(0) * es + layer * pool.k.stride(1) * es
    slab_bytes = page_size * head_dim * es
    sink = torch.zeros(8 * 3, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    offs_dev = torch.from_numpy(offs).to(dev)
    cnt_dev = torch.from_numpy(counts).to(dev)
    _lib.call("kunserve_decode_slab_probe", pool.k.data_ptr(), pool.v.data_ptr(),
              offs_dev.data_ptr(), cnt_dev.data_ptr(), 8, max_slabs, pool.k.stride(2) * es, 3,
              slab_bytes, sink.data_ptr(), stream)
    torch.cuda.synchronize()
    kw = pool.k.cpu().numpy().view(np.uint32)
    vw = pool.v.cpu().numpy().view(np.uint32)
    want = np.zeros(24, dtype=np.uint32)
    for i, n in enumerate(used):
        for h in range(3):
            x = np.uint32(0)
            for p in pages[i, :n]:
                x ^= np.bitwise_xor.reduce(kw[p, layer, h].reshape(-1))
                x ^= np.bitwise_xor.reduce(vw[p, layer, h].reshape(-1))
            want[i * 3 + h] = x
    assert np.array_equal(sink.cpu().numpy().view(np.uint32), want)
    with pytest.raises(_lib.KunserveError):
        _lib.call("kunserve_decode_slab_probe", pool.k.data_ptr(), pool.v.data_ptr(),
                  offs_dev.data_ptr(), cnt_dev.data_ptr(), 8, max_slabs, 0, 3, 1000,
                  sink.data_ptr(), stream)
    with pytest.raises(_lib.KunserveError, match="multiple of 8"):
        _lib.call("kunserve_decode_slab_probe", pool.k.data_ptr(), pool.v.data_ptr(),
                  offs_dev.data_ptr(), cnt_dev.data_ptr(), 4, max_slabs, 0, 3, slab_bytes,
                  sink.data_ptr(), stream)

