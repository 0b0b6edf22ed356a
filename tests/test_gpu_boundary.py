"""The drop-in boundary on the GPU: what the C ABI does with bad input, the
use_tensor_cores mode of pforward, and that the Python shim never makes the
host wait for the device.

* Page ids outside the pool reach kunserve_paged_decode and
  kunserve_paged_prefill unchecked (the PageTable here does not validate),
  and every kernel must drop the tokens of such a page from the softmax:
  the output equals the oracle's on the table without that page.
* A non-positive or non-finite sm_scale is rejected (EINVAL), since the
  kernels' masking relies on scale > 0.
* kunserve/flash_backend.py:2460-2462 flags every row as prefill under
  --use-tensor-cores; a pforward step in that mode must append at the A3
  positions and attend as the oracle does.
* pforward, AttentionStep.run, local_copy_blocks and kv_exchange_pack run
  under torch.cuda.set_sync_debug_mode("error"): stream-ordered, as the
  reference's swap/step overlap needs (kunserve/worker.py:289-296).
"""
import math

import numpy as np
import pytest
import torch

from kunserve_amd import (DecodePlan, LlamaOp, PrefillPlan, paged_decode, paged_prefill)
from kunserve_amd._lib import EINVAL, KunserveError
from oracle import paged_attention_ref as ref

from helpers import (ATOL, ATOL_BF16, compact_for_oracle, max_abs, random_pool, random_tensor,
                     table_from_csr, to_numpy)

pytestmark = pytest.mark.gpu


def csr(rows):
    indptr = np.concatenate([[0], np.cumsum([len(r) for r in rows])]).astype(np.int32)
    indices = np.concatenate(rows).astype(np.int32) if rows else np.zeros(0, np.int32)
    return indptr, indices


def without_bad_pages(rows, kv, num_pages, ps):
    """The table the oracle sees: bad pages removed, each taking its
    page_size tokens with it (the bad pages are whole pages)."""
    good_rows, good_kv = [], []
    for pages, n in zip(rows, kv):
        good = [p for p in pages if 0 <= p < num_pages]
        good_rows.append(good)
        good_kv.append(n - ps * (len(pages) - len(good)))
    return good_rows, np.asarray(good_kv, dtype=np.int32)


@pytest.mark.parametrize("hq,hkv", [(4, 4), (16, 2)])
@pytest.mark.parametrize("bad", [-7, 1 << 20])
def test_decode_drops_tokens_of_bad_page_ids(device, hq, hkv, bad):
    """One decode call straight through the C ABI with out-of-range ids:
    row 1 has one in the middle, row 2 has nothing but bad pages. VALU
    kernel (1 q head per KV head) and MFMA kernel (8)."""
    rng = np.random.default_rng(1)
    npg, ps = 96, 16
    kv = np.array([100, 333, 64, 700], dtype=np.int32)
    perm = rng.permutation(npg)
    rows, at = [], 0
    for n in (kv + ps - 1) // ps:
        rows.append(perm[at:at + n].tolist())
        at += n
    rows[1][5] = bad
    rows[2] = [bad] * 4
    indptr, indices = csr(rows)
    pool = random_pool(npg, 2, hkv, ps, 128, device, 3)
    q = random_tensor((4, hq, 128), device, 4)
    for part in (0, 256):
        plan = DecodePlan(kv, hq, hkv, device, part_tokens=part)
        out = paged_decode(pool, 1, table_from_csr(indptr, indices, kv, device), q, plan)
        torch.cuda.synchronize()
        good_rows, good_kv = without_bad_pages(rows, kv, npg, ps)
        gi, gx = csr(good_rows)
        want = ref.decode_attention(to_numpy(q), to_numpy(pool.k), to_numpy(pool.v), 1, gi, gx,
                                    good_kv, 1 / math.sqrt(128))
        assert max_abs(out, want) <= ATOL
        assert not out[2].float().abs().max().item()     # nothing visible: zeros


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hd", [64, 128, 256])
@pytest.mark.parametrize("ps,long_row", [(16, False), (4, True)])
def test_prefill_drops_tokens_of_bad_page_ids(device, ps, long_row, hd, dtype):
    """Prefill rows with a bad id among their prefix pages (staged page ids,
    and rows too long to stage them at page size 4), on each prefill kernel
    (warp-specialised at head_dim 64 and 128, whose loader lanes differ, and
    the 4-wave kernel at 256), fp16 and bf16, whole and split KV ranges. The
    kept tokens keep their causal order, so the oracle runs on the table
    without the page."""
    rng = np.random.default_rng(5)
    hq, hkv = 8, 2
    q_lens = np.array([40, 100], dtype=np.int32)
    prefix = np.array([64, 8960 if long_row else 200], dtype=np.int32)
    kv = prefix + q_lens
    need = (kv + ps - 1) // ps
    npg = int(need.sum()) + 8
    perm = rng.permutation(npg)
    rows, at = [], 0
    for n in need:
        rows.append(perm[at:at + n].tolist())
        at += n
    rows[0][1] = -3
    rows[1][3] = npg + 11
    indptr, indices = csr(rows)
    q_indptr = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    pool = random_pool(npg, 1, hkv, ps, hd, device, 6, dtype=dtype)
    q = random_tensor((int(q_lens.sum()), hq, hd), device, 7, dtype=dtype)
    qi = torch.from_numpy(q_indptr).to(device)
    tol = ATOL if dtype == torch.float16 else ATOL_BF16
    good_rows, good_kv = without_bad_pages(rows, kv, npg, ps)
    gi, gx = csr(good_rows)
    want = ref.prefill_attention(to_numpy(q), q_indptr, to_numpy(pool.k), to_numpy(pool.v),
                                 0, gi, gx, good_kv, 1 / math.sqrt(hd))
    for cus in (None, 1024):          # whole rows, and KV ranges split over workgroups
        plan = PrefillPlan(q_indptr, kv, hq, hkv, device, num_cus=cus, head_dim=hd)
        if cus is not None:
            assert plan.info.num_merge > 0
        out = paged_prefill(pool, 0, table_from_csr(indptr, indices, kv, device), qi, q, plan)
        torch.cuda.synchronize()
        assert max_abs(out, want) <= tol, (cus, max_abs(out, want))


@pytest.mark.parametrize("scale", [0.0, -0.088, float("nan"), float("inf")])
def test_bad_sm_scale_is_rejected(device, scale):
    pool = random_pool(8, 1, 2, 16, 128, device, 8)
    kv = np.array([20], dtype=np.int32)
    table = table_from_csr(np.array([0, 2], np.int32), np.array([3, 5], np.int32), kv, device)
    q = random_tensor((1, 2, 128), device, 9)
    with pytest.raises(KunserveError) as e:
        paged_decode(pool, 0, table, q, DecodePlan(kv, 2, 2, device), sm_scale=scale)
    assert e.value.code == EINVAL
    qi = torch.tensor([0, 1], dtype=torch.int32, device=device)
    with pytest.raises(KunserveError) as e:
        paged_prefill(pool, 0, table, qi, q, PrefillPlan(np.array([0, 1]), kv, 2, 2, device),
                      sm_scale=scale)
    assert e.value.code == EINVAL


def test_pforward_with_tensor_cores(device):
    """Every row flagged as prefill (kunserve/request.py:667-670), with the
    rows' real stages passed as is_context_stage: decode rows (one token,
    first = prompt_len + output_len) append at first - 1 inside the
    ceil(first / 16) blocks the block manager holds; chunk rows at
    [first, first + q_len). The last row is a decode row its page count
    settles (first 64 on 4 pages); the same step without the stages
    raises."""
    op = LlamaOp(256, 2, 8, 4, 16, 128, 1, 1, 8, 4096, 4096, 1, device, use_tensor_cores=True)
    op.pool.k.copy_(random_tensor(op.pool.k.shape, device, 11))
    op.pool.v.copy_(random_tensor(op.pool.v.shape, device, 12))
    rng = np.random.default_rng(13)
    perm = rng.permutation(256)
    first = [32, 77, 0, 1, 64]
    q_lens = [100, 1, 20, 1, 1]
    stage = [1, 0, 1, 0, 0]
    flags = [1] * 5
    kv = ref.kv_lens_for_step(first, q_lens, flags, True, stage)
    assert kv.tolist() == [132, 77, 20, 1, 64]
    need = (kv + 15) // 16           # exactly the blocks allocated (block_manager.py:493-500)
    pages, at = [], 0
    for n in need:
        pages.append(perm[at:at + n].tolist())
        at += n
    T = sum(q_lens)
    tokens = [[0] * n for n in q_lens]
    with pytest.raises(ValueError, match="is_context_stage"):
        op.pforward(5, T, 256, 0, 2, tokens, first, flags, pages)
    step = op.pforward(5, T, 256, 0, 2, tokens, first, flags, pages, is_context_stage=stage)
    assert step.decode is not None and step.decode.rows.tolist() == [1, 3, 4]
    q = random_tensor((T, 8, 128), device, 14)
    k = random_tensor((T, 4, 128), device, 15)
    v = random_tensor((T, 4, 128), device, 16)
    kh, vh = to_numpy(op.pool.k), to_numpy(op.pool.v)
    out = step.run(1, q, k, v)
    torch.cuda.synchronize()
    q_indptr = np.concatenate([[0], np.cumsum(q_lens)])
    indptr, indices = csr(pages)
    ref.append_kv(kh, vh, 1, indptr, indices, kv, q_indptr, to_numpy(k), to_numpy(v))
    assert np.array_equal(to_numpy(op.pool.k).view(np.int16), kh.view(np.int16))
    assert np.array_equal(to_numpy(op.pool.v).view(np.int16), vh.view(np.int16))
    want = ref.prefill_attention(to_numpy(q), q_indptr, kh, vh, 1, indptr, indices, kv,
                                 1 / math.sqrt(128))
    assert max_abs(out, want) <= ATOL


def test_tensor_cores_lifecycle_with_one_token_tail_chunk(device):
    """Whole request lifecycles under --use-tensor-cores with is_context_stage
    (kunserve/request.py:368-462,654-670): a 513-token prompt in chunks of
    512 ends in a one-token chunk at first index 512; beside it run a
    1040-token prompt (chunks 512, 512, 16) and a 20-token one. Every step
    goes through LlamaOp.pforward (every row flagged) and matches the
    oracle: the appends bit for bit, attention to ATOL. At the end each
    request's cached K/V, read back position by position through its table,
    is exactly the sequence of k/v rows it was given: every position was
    appended once, in order."""
    from lifecycle import Request

    ps, hq, hkv, d, chunk = 16, 8, 4, 128, 512
    op = LlamaOp(512, 1, hq, hkv, ps, d, 1, 1, 8, 4096, 4096, 1, device, use_tensor_cores=True)
    op.pool.k.zero_()
    op.pool.v.zero_()
    reqs = [Request(513, chunk), Request(1040, chunk), Request(20, chunk)]
    rng = np.random.default_rng(21)
    perm = rng.permutation(512).tolist()
    blocks = [perm[0:40], perm[40:120], perm[120:130]]     # enough for 600 / 1100 / 80 tokens
    given_k = [[] for _ in reqs]
    given_v = [[] for _ in reqs]
    kh, vh = to_numpy(op.pool.k), to_numpy(op.pool.v)
    seed = 100
    tail_seen = False
    for step_no in range(6):
        args = [r.step_args(True, ps) for r in reqs]
        first = [a[0] for a in args]
        q_lens = [a[1] for a in args]
        flags = [a[2] for a in args]
        stage = [a[3] for a in args]
        # a context row's table is cut to its chunk's end (block_manager.py:786-795)
        pages = [blocks[i][:a[4]] for i, a in enumerate(args)]
        tail_seen |= any(s == 1 and ql == 1 and f > 0 for s, ql, f in zip(stage, q_lens, first))
        T = sum(q_lens)
        step = op.pforward(len(reqs), T, 512, 0, 1, [[0] * n for n in q_lens], first, flags,
                           pages, is_context_stage=stage)
        q = random_tensor((T, hq, d), device, seed)
        k = random_tensor((T, hkv, d), device, seed + 1)
        v = random_tensor((T, hkv, d), device, seed + 2)
        seed += 3
        out = step.run(0, q, k, v)
        torch.cuda.synchronize()
        kv = ref.kv_lens_for_step(first, q_lens, flags, True, stage)
        q_indptr = np.concatenate([[0], np.cumsum(q_lens)])
        indptr, indices = csr(pages)
        ref.append_kv(kh, vh, 0, indptr, indices, kv, q_indptr, to_numpy(k), to_numpy(v))
        assert np.array_equal(to_numpy(op.pool.k).view(np.int16), kh.view(np.int16)), step_no
        assert np.array_equal(to_numpy(op.pool.v).view(np.int16), vh.view(np.int16)), step_no
        want = ref.prefill_attention(to_numpy(q), q_indptr, kh, vh, 0, indptr, indices, kv,
                                     1 / math.sqrt(d))
        assert max_abs(out, want) <= ATOL, step_no
        for i in range(len(reqs)):
            given_k[i].append(to_numpy(k[q_indptr[i]:q_indptr[i + 1]]))
            given_v[i].append(to_numpy(v[q_indptr[i]:q_indptr[i + 1]]))
            reqs[i].finish_step()
    assert tail_seen
    kp, vp = to_numpy(op.pool.k), to_numpy(op.pool.v)
    for i, r in enumerate(reqs):
        n = r.prompt_len + r.outputs - 1       # positions written (the last decode's token too)
        pos = np.arange(n)
        pg = np.asarray(blocks[i])[pos // ps]
        got_k = kp[pg, 0, :, pos % ps]          # [n, hkv, d]
        got_v = vp[pg, 0, :, pos % ps]
        want_k = np.concatenate(given_k[i])
        want_v = np.concatenate(given_v[i])
        assert want_k.shape[0] == n, (i, want_k.shape, n)
        assert np.array_equal(got_k.view(np.int16), want_k.view(np.int16)), i
        assert np.array_equal(got_v.view(np.int16), want_v.view(np.int16)), i

def test_reference_constructor_call(device):
    """The reference's own constructor call (kunserve/models.py:52-65: 12
    positional ints, Llama-2-7B values at a small page count) through
    torch.classes.gpt_ops.LlamaOp, then a decode step of pforward's 13
    arguments (kunserve/worker.py:298-312) against the oracle."""
    op = torch.classes.gpt_ops.LlamaOp(64, 2, 32, 32, 16, 128, 11008, 32000, 8, 4096, 4096, 1)
    assert isinstance(op, LlamaOp) and op.pool.k.device == device
    op.pool.k.copy_(random_tensor(op.pool.k.shape, device, 31))
    op.pool.v.copy_(random_tensor(op.pool.v.shape, device, 32))
    first, flags, q_lens = [37, 100], [0, 0], [1, 1]
    pages = [[3, 9, 4], [10, 11, 12, 13, 14, 15, 16]]
    step = op.pforward(2, 2, 64, 0, 2, [[0], [0]], first, flags, pages)
    q = random_tensor((2, 32, 128), device, 33)
    k = random_tensor((2, 32, 128), device, 34)
    v = random_tensor((2, 32, 128), device, 35)
    kh, vh = to_numpy(op.pool.k), to_numpy(op.pool.v)
    out = step.run(1, q, k, v)
    torch.cuda.synchronize()
    kv = ref.kv_lens_for_step(first, q_lens, flags)
    q_indptr = np.array([0, 1, 2])
    indptr, indices = csr(pages)
    ref.append_kv(kh, vh, 1, indptr, indices, kv, q_indptr, to_numpy(k), to_numpy(v))
    want = ref.decode_attention(to_numpy(q), kh, vh, 1, indptr, indices, kv, 1 / math.sqrt(128))
    assert max_abs(out, want) <= ATOL


def test_shim_never_waits_for_the_device(device):
    """A mixed pforward step, its per-layer run, a local block copy and a
    kv_exchange pack, all with torch's sync debug mode set to raise."""
    op = LlamaOp(128, 2, 8, 2, 16, 128, 1, 1, 8, 4096, 4096, 1, device)
    op.pool.k.copy_(random_tensor(op.pool.k.shape, device, 21))
    op.pool.v.copy_(random_tensor(op.pool.v.shape, device, 22))
    first, flags, q_lens = [40, 300, 7], [1, 0, 1], [60, 1, 9]
    kv = ref.kv_lens_for_step(first, q_lens, flags)
    need = (kv + 15) // 16
    perm = np.random.default_rng(23).permutation(100)
    pages, at = [], 0
    for n in need:
        pages.append(perm[at:at + n].tolist())
        at += n
    T = sum(q_lens)
    q = random_tensor((T, 8, 128), device, 24)
    k = random_tensor((T, 2, 128), device, 25)
    v = random_tensor((T, 2, 128), device, 26)
    kh, vh = to_numpy(op.pool.k), to_numpy(op.pool.v)
    torch.cuda.synchronize()
    mode = torch.cuda.get_sync_debug_mode()
    torch.cuda.set_sync_debug_mode("error")
    try:
        step = op.pforward(3, T, 128, 0, 2, [[0] * n for n in q_lens], first, flags, pages)
        out = step.run(0, q, k, v)
        op.local_copy_blocks(128, [120, 121], [122, 123])
        scratch = op.kv_exchange_pack([101, 102, 103], 0, 2)
    finally:
        torch.cuda.set_sync_debug_mode(mode)
    torch.cuda.synchronize()
    q_indptr = np.concatenate([[0], np.cumsum(q_lens)])
    indptr, indices = csr(pages)
    ref.append_kv(kh, vh, 0, indptr, indices, kv, q_indptr, to_numpy(k), to_numpy(v))
    want = ref.prefill_attention(to_numpy(q), q_indptr, kh, vh, 0, indptr, indices, kv,
                                 1 / math.sqrt(128))
    assert max_abs(out, want) <= ATOL
    assert torch.equal(op.pool.k[122:124].view(torch.int16), op.pool.k[120:122].view(torch.int16))
    packed = ref.kv_pack(to_numpy(op.pool.k), to_numpy(op.pool.v), 0, 2, [101, 102, 103])
    assert np.array_equal(to_numpy(scratch)[:packed.size].reshape(packed.shape).view(np.int16),
                          packed.view(np.int16))
