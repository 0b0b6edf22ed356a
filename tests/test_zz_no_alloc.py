"""kunserve_paged_decode_noalloc (decode whose split partials live in a
static device array) against kunserve_paged_decode with a caller workspace,
both called through the C ABI: bit-exact, on two calls in a row with the
second smaller, and with plans that split rows (so the static array is
used). A plan needing more than the array fails on the host with ENOSPC."""
import ctypes

import numpy as np
import pytest
import torch

from kunserve_amd import DecodePlan, _lib
from kunserve_amd.paged_kv import _tensor3

from helpers import random_pool, random_tensor, table_from_csr

pytestmark = pytest.mark.gpu


def _stream(device):
    return torch.cuda.current_stream(device).cuda_stream


def _decode_both(pool, table, q, plan, device):
    hq = q.shape[1]
    ws_bytes = plan.workspace_bytes(pool.head_dim)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    ref_out = torch.full_like(q, float("nan"))
    out = torch.full_like(q, float("nan"))
    qd, od, rd = _tensor3(q), _tensor3(out), _tensor3(ref_out)
    scale = ctypes.c_float(1 / 128 ** 0.5)
    _lib.call("kunserve_paged_decode", pool.desc(), 1, table.desc(), None, ctypes.byref(qd),
              ctypes.byref(rd), hq, scale, plan.plan.data_ptr(), ctypes.byref(plan.info),
              ws.data_ptr(), ws.numel(), _stream(device))
    _lib.call("kunserve_paged_decode_noalloc", pool.desc(), 1, table.desc(), None,
              ctypes.byref(qd),
              ctypes.byref(od), hq, scale, plan.plan.data_ptr(), ctypes.byref(plan.info),
              _stream(device))
    torch.cuda.synchronize()
    return ref_out, out


def _rows(rng, kv, npg, ps):
    need = (kv + ps - 1) // ps
    indptr = np.concatenate([[0], np.cumsum(need)]).astype(np.int32)
    indices = rng.permutation(npg)[:indptr[-1]].astype(np.int32)
    return indptr, indices


@pytest.mark.parametrize("hq,hkv", [(32, 32), (32, 4)])
def test_noalloc_decode_equals_workspace_decode(device, hq, hkv):
    rng = np.random.default_rng(hq + hkv)
    npg, ps = 2048, 16
    pool = random_pool(npg, 2, hkv, ps, 128, device, 3)
    for kv in (np.array([3000, 17, 900, 4500, 1, 0, 2600], dtype=np.int32),
               np.array([700, 260], dtype=np.int32)):           # second call: smaller
        indptr, indices = _rows(rng, kv, npg, ps)
        table = table_from_csr(indptr, indices, kv, device)
        q = random_tensor((len(kv), hq, 128), device, int(kv.sum()))
        plan = DecodePlan(kv, hq, hkv, device, part_tokens=256)
        assert plan.info.num_slots > 0            # rows split: the static partials are used
        want, got = _decode_both(pool, table, q, plan, device)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))


def test_noalloc_decode_rejects_plans_beyond_its_scratch(device):
    limit = _lib.lib().kunserve_paged_decode_noalloc_max_bytes()
    assert limit == 32 << 20
    hq, hkv = 64, 64
    kv = np.full(96, 8192, dtype=np.int32)
    plan = DecodePlan(kv, hq, hkv, device, part_tokens=256)
    assert plan.workspace_bytes(128) > limit
    pool = random_pool(8, 2, hkv, 16, 128, device, 4)
    # a real table (every row on page 0 of the pool), so that a call past the
    # host check would still read only pool memory
    per_row = (8192 + 15) // 16
    table = table_from_csr(np.arange(97, dtype=np.int32) * per_row,
                           np.zeros(96 * per_row, np.int32), kv, device)
    q = random_tensor((96, hq, 128), device, 5)
    qd, od = _tensor3(q), _tensor3(torch.empty_like(q))
    with pytest.raises(_lib.KunserveError) as e:
        _lib.call("kunserve_paged_decode_noalloc", pool.desc(), 1, table.desc(), None,
                  ctypes.byref(qd), ctypes.byref(od), hq, ctypes.c_float(0.088),
                  plan.plan.data_ptr(), ctypes.byref(plan.info), _stream(device))
    assert e.value.code == _lib.ENOSPC
