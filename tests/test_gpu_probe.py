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
