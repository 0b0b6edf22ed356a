"""K/V append (bit-exact) and chunked-prefill attention (max-abs <= 2e-3)
on the GPU vs the CPU oracle, plus the pforward attention stage."""
import math

import numpy as np
import pytest
import torch

from kunserve_amd import (AttentionStep, LlamaOp, PrefillPlan, append_kv, paged_decode,
                          paged_prefill, workloads, DecodePlan)
from oracle import paged_attention_ref as ref

from helpers import ATOL, compact_for_oracle, max_abs, random_pool, random_tensor, table_from_csr

pytestmark = pytest.mark.gpu


def make_rows(rng, q_lens, prefixes, ps, npg):
    kv = np.asarray(prefixes) + np.asarray(q_lens)
    need = (kv + ps - 1) // ps
    indptr = np.concatenate([[0], np.cumsum(need)]).astype(np.int32)
    indices = rng.permutation(npg)[:indptr[-1]].astype(np.int32)
    q_indptr = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    return kv.astype(np.int32), indptr, indices, q_indptr


def test_append_bit_exact(device):
    rng = np.random.default_rng(0)
    ps, npg, hkv, d = 16, 64, 4, 128
    q_lens, prefixes = [5, 1, 40, 16], [0, 33, 7, 16]
    kv, indptr, indices, q_indptr = make_rows(rng, q_lens, prefixes, ps, npg)
    pool = random_pool(npg, 3, hkv, ps, d, device, 1)
    k0, v0 = pool.k.cpu().numpy(), pool.v.cpu().numpy()
    T = int(q_indptr[-1])
    kn, vn = random_tensor((T, hkv, d), device, 2), random_tensor((T, hkv, d), device, 3)
    table = table_from_csr(indptr, indices, kv, device)
    append_kv(pool, 2, table, torch.from_numpy(q_indptr).to(device), kn, vn)
    torch.cuda.synchronize()
    ref.append_kv(k0, v0, 2, indptr, indices, kv, q_indptr, kn.cpu().numpy(), vn.cpu().numpy())
    assert np.array_equal(pool.k.cpu().numpy().view(np.int16), k0.view(np.int16))
    assert np.array_equal(pool.v.cpu().numpy().view(np.int16), v0.view(np.int16))


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("num_rows,hkv", [(5, 8), (70, 1), (70, 8)])
def test_append_tiles_rows_and_skipped_tokens(device, d, num_rows, hkv):
    """The append kernel's token tiles against the oracle: fewer than 64
    rows (rows found by a ballot over q_indptr) and 70 rows (binary search),
    empty rows, tiles that straddle rows and pages, step tokens no row owns
    (num_tokens > q_indptr[-1]), and page ids outside the pool, whose tokens
    are dropped (the oracle writes them to a spare page that the check then
    ignores)."""
    rng = np.random.default_rng(num_rows * 1000 + d + hkv)
    ps, layers = 16, 2
    q_lens = rng.integers(0, 40, num_rows)
    q_lens[::7] = 0                                    # empty rows
    prefixes = rng.integers(0, 100, num_rows)
    kv = (prefixes + q_lens).astype(np.int32)
    need = (kv + ps - 1) // ps
    npg = int(need.sum()) + 4
    indptr = np.concatenate([[0], np.cumsum(need)]).astype(np.int32)
    indices = rng.permutation(npg)[:indptr[-1]].astype(np.int32)
    bad = rng.choice(indptr[-1], size=3, replace=False)
    indices[bad[0]], indices[bad[1]], indices[bad[2]] = -1, npg, npg + 1000
    q_indptr = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    T = int(q_indptr[-1]) + 9                          # 9 trailing tokens no row owns
    pool = random_pool(npg, layers, hkv, ps, d, device, 1)
    kn, vn = random_tensor((T, hkv, d), device, 2), random_tensor((T, hkv, d), device, 3)
    k0, v0 = pool.k.cpu().numpy(), pool.v.cpu().numpy()
    append_kv(pool, 1, table_from_csr(indptr, indices, kv, device),
              torch.from_numpy(q_indptr).to(device), kn, vn)
    torch.cuda.synchronize()
    spare = np.concatenate([k0, k0[:1]]), np.concatenate([v0, v0[:1]])
    ids = np.where((indices >= 0) & (indices < npg), indices, npg).astype(np.int32)
    ref.append_kv(spare[0], spare[1], 1, indptr, ids, kv, q_indptr, kn.cpu().numpy(),
                  vn.cpu().numpy())
    assert np.array_equal(pool.k.cpu().numpy().view(np.int16), spare[0][:npg].view(np.int16))
    assert np.array_equal(pool.v.cpu().numpy().view(np.int16), spare[1][:npg].view(np.int16))


def run_prefill(pool, layer, q_lens, kv, indptr, indices, q_indptr, hq, device, seed):
    T = int(q_indptr[-1])
    q = random_tensor((T, hq, pool.head_dim), device, seed)
    table = table_from_csr(indptr, indices, kv, device)
    plan = PrefillPlan(q_indptr, kv, hq, pool.num_kv_heads, device, head_dim=pool.head_dim)
    out = paged_prefill(pool, layer, table, torch.from_numpy(q_indptr).to(device), q, plan)
    torch.cuda.synchronize()
    return q, out


def oracle_prefill(pool, layer, q, q_indptr, indptr, indices, kv, rows=None):
    """The numpy oracle's prefill of every row, or of the rows listed (their
    q rows concatenated, in that order)."""
    scale = 1.0 / math.sqrt(pool.head_dim)
    if rows is None:
        k, v, ip, ix = compact_for_oracle(pool, layer, indptr, indices)
        return ref.prefill_attention(q.cpu().numpy(), q_indptr, k, v, 0, ip, ix, kv, scale)
    k, v, ip, ix = compact_for_oracle(pool, layer, indptr, indices, rows)
    qs = torch.cat([q[int(q_indptr[b]):int(q_indptr[b + 1])] for b in rows])
    qi = np.concatenate([[0], np.cumsum([int(q_indptr[b + 1] - q_indptr[b]) for b in rows])])
    return ref.prefill_attention(qs.cpu().numpy(), qi, k, v, 0, ip, ix, np.asarray(kv)[rows],
                                 scale)


@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 2), (12, 4)])
@pytest.mark.parametrize("ps", [16, 64])
def test_prefill_matches_oracle(device, hq, hkv, ps):
    rng = np.random.default_rng(hq + ps)
    q_lens = [1, 5, 64, 127, 128, 129, 300, 512]
    prefixes = [0, 17, 0, 100, 1000, 3, 64, 2048]
    npg = 400 if ps == 16 else 120
    kv, indptr, indices, q_indptr = make_rows(rng, q_lens, prefixes, ps, npg)
    pool = random_pool(npg, 2, hkv, ps, 128, device, 5)
    q, out = run_prefill(pool, 1, q_lens, kv, indptr, indices, q_indptr, hq, device, 6)
    want = oracle_prefill(pool, 1, q, q_indptr, indptr, indices, kv)
    assert max_abs(out, want) <= ATOL


@pytest.mark.parametrize("head_dim", [64, 256])
@pytest.mark.parametrize("hq,hkv", [(8, 8), (8, 2)])
@pytest.mark.parametrize("cus", [None, 1024])
def test_prefill_head_dims_match_oracle(device, head_dim, hq, hkv, cus):
    """head_dim 64 (8 waves, two per SIMD) and 256 (4 waves of 128-row
    tiles, one per SIMD): whole KV ranges and, with a plan made for 1024
    CUs, split ones plus the merge; ragged rows with prefixes."""
    rng = np.random.default_rng(head_dim + hq + hkv)
    q_lens = [1, 5, 64, 127, 128, 129, 300, 512]
    prefixes = [0, 17, 0, 100, 1000, 3, 64, 2048]
    kv, indptr, indices, q_indptr = make_rows(rng, q_lens, prefixes, 16, 400)
    pool = random_pool(400, 2, hkv, 16, head_dim, device, 50 + head_dim)
    q = random_tensor((int(q_indptr[-1]), hq, head_dim), device, 51)
    table = table_from_csr(indptr, indices, kv, device)
    plan = PrefillPlan(q_indptr, kv, hq, hkv, device, num_cus=cus, head_dim=head_dim)
    assert plan.info.tile_q == (128 if head_dim == 256 else 256)
    if cus == 1024:
        assert plan.info.num_merge > 0
    out = paged_prefill(pool, 1, table, torch.from_numpy(q_indptr).to(device), q, plan)
    torch.cuda.synchronize()
    want = oracle_prefill(pool, 1, q, q_indptr, indptr, indices, kv)
    assert max_abs(out, want) <= ATOL


@pytest.mark.parametrize("head_dim", [64, 256])
def test_prefill_head_dims_long_row_unstaged_ids(device, head_dim):
    """A row with more pages than the kernel stages in LDS (page size 4,
    9000 cached tokens) reads its page ids from the table, at head_dim 64
    and 256."""
    rng = np.random.default_rng(head_dim)
    q_lens, prefixes = [100, 40], [8900, 30]
    kv, indptr, indices, q_indptr = make_rows(rng, q_lens, prefixes, 4, 2400)
    pool = random_pool(2400, 1, 2, 4, head_dim, device, 60)
    q, out = run_prefill(pool, 0, q_lens, kv, indptr, indices, q_indptr, 4, device, 61)
    want = oracle_prefill(pool, 0, q, q_indptr, indptr, indices, kv)
    assert max_abs(out, want) <= ATOL


@pytest.mark.parametrize("head_dim", [64, 128, 256])
def test_prefill_large_scores_match_oracle(device, head_dim):
    """q ~ N(0, 8^2): scores span tens of log2 units, so the lazy running max
    moves many times and the softmax is sharp. The scores must keep fp32
    accuracy: rounding a pre-scaled q to fp16 (scale folded into q) put
    errors of 1e-2 into these outputs."""
    rng = np.random.default_rng(head_dim + 7)
    q_lens, prefixes = [64, 300, 512], [0, 100, 700]
    kv, indptr, indices, q_indptr = make_rows(rng, q_lens, prefixes, 16, 120)
    pool = random_pool(120, 1, 4, 16, head_dim, device, 70)
    pool.v.mul_(0.5)
    q = random_tensor((int(q_indptr[-1]), 8, head_dim), device, 71, scale=8.0)
    table = table_from_csr(indptr, indices, kv, device)
    plan = PrefillPlan(q_indptr, kv, 8, 4, device, head_dim=head_dim)
    out = paged_prefill(pool, 0, table, torch.from_numpy(q_indptr).to(device), q, plan)
    torch.cuda.synchronize()
    want = oracle_prefill(pool, 0, q, q_indptr, indptr, indices, kv)
    assert max_abs(out, want) <= ATOL


def test_prefill_plan_for_another_head_dim_is_rejected(device):
    from kunserve_amd._lib import EINVAL, KunserveError

    rng = np.random.default_rng(3)
    kv, indptr, indices, q_indptr = make_rows(rng, [10], [5], 16, 8)
    pool = random_pool(8, 1, 2, 16, 64, device, 62)
    q = random_tensor((10, 2, 64), device, 63)
    plan = PrefillPlan(q_indptr, kv, 2, 2, device)          # made for head_dim 128
    with pytest.raises(KunserveError) as e:
        paged_prefill(pool, 0, table_from_csr(indptr, indices, kv, device),
                      torch.from_numpy(q_indptr).to(device), q, plan)
    assert e.value.code == EINVAL


@pytest.mark.parametrize("ps", [16, 64])
def test_prefill_split_kv_matches_oracle(device, ps):
    """Split KV ranges (a plan made for 1024 CUs splits every tile of this
    small batch) merge to the oracle and to the unsplit result."""
    rng = np.random.default_rng(40 + ps)
    q_lens = [1, 77, 256, 300, 512]
    prefixes = [700, 0, 1500, 33, 2048]
    npg = 600 if ps == 16 else 160
    kv, indptr, indices, q_indptr = make_rows(rng, q_lens, prefixes, ps, npg)
    pool = random_pool(npg, 1, 4, ps, 128, device, 41)
    T = int(q_indptr[-1])
    q = random_tensor((T, 8, 128), device, 42)
    table = table_from_csr(indptr, indices, kv, device)
    qi = torch.from_numpy(q_indptr).to(device)
    split = PrefillPlan(q_indptr, kv, 8, 4, device, num_cus=1024)
    assert split.info.num_merge > 0 and split.info.kv_chunk >= 256
    whole = PrefillPlan(q_indptr, kv, 8, 4, device, num_cus=1)
    assert whole.info.num_merge == 0
    out_s = paged_prefill(pool, 0, table, qi, q, split)
    out_w = paged_prefill(pool, 0, table, qi, q, whole)
    torch.cuda.synchronize()
    assert max_abs(out_s, out_w.float()) <= 1e-3
    want = oracle_prefill(pool, 0, q, q_indptr, indptr, indices, kv)
    assert max_abs(out_s, want) <= ATOL


@pytest.mark.parametrize("cus", [1, 1024])
def test_prefill_graph_replays_and_repeats(device, cus):
    """Prefill (whole items with one CU's plan; split KV ranges and the merge
    with 1024 CUs' plan) captured in a HIP graph gives the eager result bit
    for bit on every replay, with eager launches and synchronisation between
    replays; repeated eager launches are bit-identical too."""
    rng = np.random.default_rng(70)
    q_lens, prefixes = [1, 77, 256, 300, 512], [700, 0, 1500, 33, 2048]
    kv, indptr, indices, q_indptr = make_rows(rng, q_lens, prefixes, 16, 600)
    pool = random_pool(600, 1, 4, 16, 128, device, 71)
    q = random_tensor((int(q_indptr[-1]), 8, 128), device, 72)
    table = table_from_csr(indptr, indices, kv, device)
    qi = torch.from_numpy(q_indptr).to(device)
    plan = PrefillPlan(q_indptr, kv, 8, 4, device, num_cus=cus)
    assert (plan.info.num_merge > 0) == (cus == 1024)
    ws = torch.empty(max(plan.workspace_bytes(), 1), dtype=torch.uint8, device=device)
    out = torch.empty_like(q)
    eager = paged_prefill(pool, 0, table, qi, q, plan, workspace=ws).clone()
    for _ in range(3):
        again = paged_prefill(pool, 0, table, qi, q, plan, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(again, eager)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        paged_prefill(pool, 0, table, qi, q, plan, out=out, workspace=ws)
    for r in range(4):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r}"
        paged_prefill(pool, 0, table, qi, q, plan, workspace=ws)   # eager launch between replays
        torch.cuda.synchronize()
    want = oracle_prefill(pool, 0, q, q_indptr, indptr, indices, kv)
    assert max_abs(eager, want) <= ATOL


@pytest.mark.parametrize("ps", [4, 256])
def test_prefill_long_rows_beyond_staged_page_ids(device, ps):
    """A row with more pages than a workgroup stages in LDS (2048) takes the
    global page-id lookup; page size 256 is the reference's default. Both
    against the oracle."""
    rng = np.random.default_rng(60 + ps)
    q_lens = [64, 3, 130] if ps == 4 else [64, 3, 300]
    prefixes = [9000, 50, 8500] if ps == 4 else [9000, 50, 700]
    npg = 4600 if ps == 4 else 90
    kv, indptr, indices, q_indptr = make_rows(rng, q_lens, prefixes, ps, npg)
    if ps == 4:
        assert (indptr[1:] - indptr[:-1]).max() > 2048   # the unstaged path runs
    pool = random_pool(npg, 1, 2, ps, 128, device, 61)
    q, out = run_prefill(pool, 0, q_lens, kv, indptr, indices, q_indptr, 4, device, 62)
    want = oracle_prefill(pool, 0, q, q_indptr, indptr, indices, kv)
    assert max_abs(out, want) <= ATOL


def test_prefill_one_token_rows_equal_decode(device):
    """A one-token prefill row is a decode row (use_tensor_cores path)."""
    rng = np.random.default_rng(7)
    q_lens, prefixes = [1] * 6, [0, 15, 16, 300, 1000, 2047]
    kv, indptr, indices, q_indptr = make_rows(rng, q_lens, prefixes, 16, 300)
    pool = random_pool(300, 1, 8, 16, 128, device, 8)
    q, out = run_prefill(pool, 0, q_lens, kv, indptr, indices, q_indptr, 8, device, 9)
    table = table_from_csr(indptr, indices, kv, device)
    dec = paged_decode(pool, 0, table, q, DecodePlan(kv, 8, 8, device))
    assert max_abs(out, dec) <= 1e-3


def test_chunked_prefill_workload_every_step(device):
    """The 16-sequence chunked-prefill workload (prompts U[512, 4096],
    prefixes U[0, 2048], chunk 512; kunserve/request.py:368-391): every step
    appends its chunk and attends, and every row of every step is checked
    against the fp32 PyTorch restatement run on the device
    (oracle.torch_cpu.prefill_attention, pinned against the numpy oracle on
    the CPU); the first and last steps are also checked in full, and one row
    of every other step, against the numpy oracle."""
    from oracle import torch_cpu

    w = workloads.chunked_prefill()
    pool = random_pool(w.num_pages, 1, w.num_kv_heads, w.page_size, w.head_dim, device, 10)
    steps = w.steps()
    assert len(steps) == 8
    for i, (rows, ql, kv) in enumerate(steps):
        pages = [w.pages[r] for r in rows]
        q_indptr = np.concatenate([[0], np.cumsum(ql)]).astype(np.int32)
        need = (kv + 15) // 16
        indptr = np.concatenate([[0], np.cumsum(need)]).astype(np.int32)
        indices = np.concatenate([p[:n] for p, n in zip(pages, need)]).astype(np.int32)
        T = int(q_indptr[-1])
        k_new = random_tensor((T, w.num_kv_heads, w.head_dim), device, 100 + i)
        v_new = random_tensor((T, w.num_kv_heads, w.head_dim), device, 200 + i)
        table = table_from_csr(indptr, indices, kv, device)
        qi = torch.from_numpy(q_indptr).to(device)
        append_kv(pool, 0, table, qi, k_new, v_new)
        q = random_tensor((T, w.num_qo_heads, w.head_dim), device, 300 + i)
        out = paged_prefill(pool, 0, table, qi, q, PrefillPlan(q_indptr, kv, w.num_qo_heads, w.num_kv_heads, device))
        want = torch_cpu.prefill_attention(q, q_indptr, pool.k, pool.v, 0, indptr, indices, kv,
                                           1 / math.sqrt(w.head_dim))
        err = float((out.float() - want).abs().max())
        assert err <= ATOL, (i, err)
        if i in (0, len(steps) - 1):
            sample = None                              # the whole step
        else:
            sample = [int(np.argmax(kv))]              # the row deepest into its prompt
        want_np = oracle_prefill(pool, 0, q, q_indptr, indptr, indices, kv, rows=sample)
        if sample is None:
            assert max_abs(out, want_np) <= ATOL, i
        else:
            b = sample[0]
            lo, hi = int(q_indptr[b]), int(q_indptr[b + 1])
            assert max_abs(out[lo:hi], want_np) <= ATOL, i


@pytest.mark.parametrize("head_size", [64, 128, 256])
def test_attention_step_mixed_batch(device, head_size):
    """One pforward step with prefill and decode rows interleaved: append of
    every row's new tokens, then decode and prefill attention."""
    op = LlamaOp(256, 2, 8, 4, 16, head_size, 1, 1, 8, 4096, 4096, 1, device)
    op.pool.k.copy_(random_tensor(op.pool.k.shape, device, 1))
    op.pool.v.copy_(random_tensor(op.pool.v.shape, device, 2))
    rng = np.random.default_rng(3)
    perm = rng.permutation(256)
    # rows: prefill chunk (first=32, 100 tokens), decode (first=77), prefill (first=0, 20),
    # decode (first=1)
    first = [32, 77, 0, 1]
    flags = [1, 0, 1, 0]
    q_lens = [100, 1, 20, 1]
    kv = [132, 77, 20, 1]
    need = [(k + 15) // 16 for k in kv]
    pages, at = [], 0
    for n in need:
        pages.append(perm[at:at + n + 1].tolist())   # one spare page, as the block manager may hold
        at += n + 1
    tokens = [list(range(n)) for n in q_lens]
    step = op.pforward(4, sum(q_lens), 256, 0, 2, tokens, first, flags, pages, 0, [], [], 0)
    T = sum(q_lens)
    q = random_tensor((T, 8, head_size), device, 4)
    k = random_tensor((T, 4, head_size), device, 5)
    v = random_tensor((T, 4, head_size), device, 6)
    k_host, v_host = op.pool.k.cpu().numpy(), op.pool.v.cpu().numpy()
    out = step.run(1, q, k, v)
    torch.cuda.synchronize()
    q_indptr = np.concatenate([[0], np.cumsum(q_lens)])
    indptr = np.concatenate([[0], np.cumsum(need)])
    indices = np.concatenate([p[:n] for p, n in zip(pages, need)])
    ref.append_kv(k_host, v_host, 1, indptr, indices, np.array(kv), q_indptr, k.cpu().numpy(),
                  v.cpu().numpy())
    assert np.array_equal(op.pool.k.cpu().numpy().view(np.int16), k_host.view(np.int16))
    want = ref.prefill_attention(q.cpu().numpy(), q_indptr, k_host, v_host, 1, indptr, indices,
                                 np.array(kv), 1 / math.sqrt(head_size))
    assert max_abs(out, want) <= ATOL
    assert step.decode is not None and step.prefill is not None


def test_pforward_validates_arguments(device):
    op = LlamaOp(16, 1, 2, 2, 16, 128, 1, 1, 8, 64, 64, 1, device)
    with pytest.raises(ValueError, match="pages"):
        op.pforward(1, 1, 16, 0, 1, [[1]], [40], [0], [[1]], 0, [], [], 0)
    with pytest.raises(IndexError):
        op.pforward(1, 1, 16, 0, 1, [[1]], [3], [0], [[16]], 0, [], [], 0)
    with pytest.raises(ValueError, match="num_tokens"):
        op.pforward(1, 2, 16, 0, 1, [[1]], [3], [0], [[1]], 0, [], [], 0)
