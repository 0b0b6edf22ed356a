"""Mixed steps in place: the decode and prefill rows of one step
(kunserve/flash_backend.py:1870-1950 batches running decodes with prefill
chunks; rows from kunserve/request.py:654-670) read q and write out where
the step's tokens lie, through the row -> token maps of
kunserve_paged_decode (q_token) and kunserve_paged_prefill (q_start).

Each subset's output equals, bit for bit, the same kernel run on compact
copies of its rows' q (the gather-and-scatter path it replaces) and matches
the oracle; tokens owned by no row keep their sentinel bits; AttentionStep
of a mixed step runs no torch gather or scatter."""
import math

import numpy as np
import pytest
import torch

from kunserve_amd import (AttentionStep, DecodePlan, LlamaOp, PrefillPlan, paged_decode,
                          paged_prefill)
from oracle import paged_attention_ref as ref

from helpers import (ATOL, ATOL_BF16, max_abs, random_pool, random_tensor, table_from_csr,
                     to_numpy)

pytestmark = pytest.mark.gpu


def csr(rows):
    indptr = np.concatenate([[0], np.cumsum([len(r) for r in rows])]).astype(np.int32)
    indices = np.concatenate(rows).astype(np.int32) if rows else np.zeros(0, np.int32)
    return indptr, indices


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hq,hkv,hd", [(8, 8, 128), (16, 2, 128), (32, 4, 128), (8, 4, 64),
                                       (8, 2, 256)])
def test_row_maps_read_and_write_in_place(device, hq, hkv, hd, dtype):
    """Six rows, prefill (P) and decode (D) interleaved: P 40 tokens on a
    30-token prefix, D at 77, P 100 on 500, D at 1, D at 3000 (split over
    partitions: the merge kernel writes through the map too), P 1 on 17.
    The step's q and out carry 5 spare tokens past its last."""
    rng = np.random.default_rng(hq * hd + hkv)
    ps = 16
    kinds = ["P", "D", "P", "D", "D", "P"]
    q_lens = np.array([40, 1, 100, 1, 1, 1])
    kv = np.array([70, 77, 600, 1, 3000, 18], dtype=np.int32)
    need = (kv + ps - 1) // ps
    npg = int(need.sum()) + 10
    perm = rng.permutation(npg)
    rows, at = [], 0
    for n in need:
        rows.append(perm[at:at + n].tolist())
        at += n
    q_indptr = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    T = int(q_indptr[-1])
    pool = random_pool(npg, 2, hkv, ps, hd, device, 3, dtype=dtype)
    q = random_tensor((T + 5, hq, hd), device, 4, dtype=dtype)
    sentinel = torch.full((T + 5, hq, hd), float("nan"), dtype=dtype, device=device)
    out = sentinel.clone()
    dec = np.array([i for i, k in enumerate(kinds) if k == "D"])
    pre = np.array([i for i, k in enumerate(kinds) if k == "P"])

    dtab = table_from_csr(*csr([rows[i] for i in dec]), kv[dec], device)
    dplan = DecodePlan(kv[dec], hq, hkv, device, part_tokens=256)
    assert dplan.info.num_merge > 0
    q_token = torch.from_numpy(q_indptr[dec].astype(np.int32)).to(device)
    paged_decode(pool, 1, dtab, q, dplan, out=out, q_token=q_token)

    pi = np.concatenate([[0], np.cumsum(q_lens[pre])]).astype(np.int32)
    ptab = table_from_csr(*csr([rows[i] for i in pre]), kv[pre], device)
    pqi = torch.from_numpy(pi).to(device)
    q_start = torch.from_numpy(q_indptr[pre].astype(np.int32)).to(device)
    for cus in (None, 1024):      # whole KV ranges, then split ranges and the merge kernel
        pplan = PrefillPlan(pi, kv[pre], hq, hkv, device, num_cus=cus, head_dim=hd)
        assert cus is None or pplan.info.num_merge > 0
        paged_prefill(pool, 1, ptab, pqi, q, pplan, out=out, q_start=q_start)
        torch.cuda.synchronize()

        # the same kernels on compact copies of the subsets' q
        dtok = torch.from_numpy(q_indptr[dec].astype(np.int64)).to(device)
        ptok = torch.from_numpy(np.concatenate(
            [np.arange(q_indptr[i], q_indptr[i + 1]) for i in pre]).astype(np.int64)).to(device)
        d_compact = paged_decode(pool, 1, dtab, q.index_select(0, dtok).contiguous(), dplan)
        p_compact = paged_prefill(pool, 1, ptab, pqi, q.index_select(0, ptok).contiguous(),
                                  pplan)
        torch.cuda.synchronize()
        assert torch.equal(out.index_select(0, dtok).view(torch.int16),
                           d_compact.view(torch.int16))
        assert torch.equal(out.index_select(0, ptok).view(torch.int16),
                           p_compact.view(torch.int16))
        assert torch.equal(out[T:].view(torch.int16), sentinel[T:].view(torch.int16))

    tol = ATOL if dtype == torch.float16 else ATOL_BF16
    indptr, indices = csr(rows)
    want = ref.prefill_attention(to_numpy(q[:T]), q_indptr, to_numpy(pool.k), to_numpy(pool.v),
                                 1, indptr, indices, kv, 1 / math.sqrt(hd))
    assert max_abs(out[:T], want) <= tol


def test_mixed_step_runs_in_place(device):
    """AttentionStep over a mixed step: the subsets carry row -> token maps
    (not per-token index lists), run() matches the oracle, and the step
    launches only this library's kernels (torch's profiler sees no gather,
    index or scatter kernel)."""
    op = LlamaOp(512, 2, 16, 4, 16, 128, 1, 1, 8, 4096, 4096, 1, device)
    op.pool.k.copy_(random_tensor(op.pool.k.shape, device, 1))
    op.pool.v.copy_(random_tensor(op.pool.v.shape, device, 2))
    rng = np.random.default_rng(3)
    perm = rng.permutation(512)
    first = [32, 700, 0, 95, 1500]
    flags = [1, 0, 1, 0, 0]
    q_lens = [300, 1, 64, 1, 1]
    kv = [332, 700, 64, 95, 1500]
    need = [(k + 15) // 16 for k in kv]
    pages, at = [], 0
    for n in need:
        pages.append(perm[at:at + n].tolist())
        at += n
    T = sum(q_lens)
    step = op.pforward(5, T, 512, 0, 2, [[0] * n for n in q_lens], first, flags, pages)
    assert step.decode.tokens.numel() == 3 and step.prefill.tokens.numel() == 2
    q = random_tensor((T, 16, 128), device, 4)
    k = random_tensor((T, 4, 128), device, 5)
    v = random_tensor((T, 4, 128), device, 6)
    kh, vh = to_numpy(op.pool.k), to_numpy(op.pool.v)
    with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CUDA]) as prof:
        out = step.run(1, q, k, v)
        torch.cuda.synchronize()
    names = [e.name for e in prof.events() if e.device_type == torch.autograd.DeviceType.CUDA]
    assert any("paged_prefill" in n for n in names) and any("paged_decode" in n for n in names)
    foreign = [n for n in names if any(w in n.lower() for w in ("index", "gather", "scatter"))]
    assert not foreign, foreign
    q_indptr = np.concatenate([[0], np.cumsum(q_lens)])
    indptr, indices = csr([p for p in pages])
    ref.append_kv(kh, vh, 1, indptr, indices, np.array(kv), q_indptr, to_numpy(k), to_numpy(v))
    want = ref.prefill_attention(to_numpy(q), q_indptr, kh, vh, 1, indptr, indices,
                                 np.array(kv), 1 / math.sqrt(128))
    assert max_abs(out, want) <= ATOL
