"""Paged decode attention on the GPU vs the CPU oracle (max-abs <= 2e-3)."""
import math

import numpy as np
import pytest
import torch

from kunserve_amd import DecodePlan, paged_decode, workloads
from oracle import paged_attention_ref as ref

from helpers import (ATOL, ATOL_BF16, compact_for_oracle, max_abs, random_pool, random_tensor,
                     table_from_csr, to_numpy, torch_decode_ref)

pytestmark = pytest.mark.gpu


def run_decode(pool, layer, indptr, indices, kv_len, hq, device, seed, part_tokens=0,
               q_scale=1.0):
    table = table_from_csr(indptr, indices, kv_len, device)
    q = random_tensor((len(kv_len), hq, pool.head_dim), device, seed, q_scale)
    plan = DecodePlan(kv_len, hq, pool.num_kv_heads, device, part_tokens=part_tokens)
    out = paged_decode(pool, layer, table, q, plan)
    torch.cuda.synchronize()
    return q, out, plan


def oracle_decode(pool, layer, indptr, indices, kv_len, q, rows=None):
    rows = np.arange(len(kv_len)) if rows is None else np.asarray(rows)
    k, v, ip, ix = compact_for_oracle(pool, 0 if pool.num_layers == 1 else layer, indptr,
                                      indices, rows)
    qn = to_numpy(q[torch.from_numpy(rows).to(q.device)])
    return ref.decode_attention(qn, k, v, 0, ip, ix, np.asarray(kv_len)[rows],
                                1.0 / math.sqrt(pool.head_dim))


def test_single_layer_decode_b8(device):
    w = workloads.single_layer_decode()
    s = 1.0 / math.sqrt(128)
    pool = random_pool(w.num_pages, 1, w.num_kv_heads, w.page_size, w.head_dim, device, 11, s)
    indptr, indices = w.csr()
    q, out, _ = run_decode(pool, 0, indptr, indices, w.kv_len, w.num_qo_heads, device, 12, 0, s)
    want = oracle_decode(pool, 0, indptr, indices, w.kv_len, q)
    assert max_abs(out, want) <= ATOL


@pytest.mark.parametrize("head_dim", [64, 128, 256])
@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 4), (64, 8)])
def test_decode_large_scores_match_oracle(device, head_dim, hq, hkv):
    """q ~ N(0, 8^2): scores span tens of log2 units (sharp softmax, many
    moves of the running max, split rows merged by log-sum-exp); the VALU
    kernel (group 1) and the MFMA kernel (groups 4, 8) keep fp32 scores."""
    rng = np.random.default_rng(head_dim + hq)
    ps, npg = 16, 400
    kv = np.array([3, 64, 300, 1000, 2500], dtype=np.int32)
    need = (kv + ps - 1) // ps
    indptr = np.concatenate([[0], np.cumsum(need)]).astype(np.int32)
    indices = rng.permutation(npg)[:indptr[-1]].astype(np.int32)
    pool = random_pool(npg, 1, hkv, ps, head_dim, device, 23)
    pool.v.mul_(0.5)
    q, out, plan = run_decode(pool, 0, indptr, indices, kv, hq, device, 24, 256, 8.0)
    assert plan.info.num_merge > 0
    want = oracle_decode(pool, 0, indptr, indices, kv, q)
    assert max_abs(out, want) <= ATOL


@pytest.mark.parametrize("head_dim", [64, 128, 256])
@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 4), (16, 2), (16, 1), (12, 4), (64, 8)])
def test_decode_heads_and_dims(device, head_dim, hq, hkv):
    rng = np.random.default_rng(hq * 1000 + hkv * 10 + head_dim)
    ps, npg = 16, 600
    kv = np.array([1, 2, 15, 16, 17, 100, 255, 256, 257, 700, 1500], dtype=np.int32)
    need = (kv + ps - 1) // ps
    perm = rng.permutation(npg)
    indptr = np.concatenate([[0], np.cumsum(need)]).astype(np.int32)
    indices = perm[:indptr[-1]].astype(np.int32)
    pool = random_pool(npg, 2, hkv, ps, head_dim, device, 21)
    q, out, _ = run_decode(pool, 1, indptr, indices, kv, hq, device, 22)
    want = oracle_decode(pool, 1, indptr, indices, kv, q)
    assert max_abs(out, want) <= ATOL


@pytest.mark.parametrize("ps", [4, 8, 32, 256])
def test_decode_page_sizes(device, ps):
    rng = np.random.default_rng(ps)
    kv = np.array([1, 3, 31, 64, 513, 2049], dtype=np.int32)
    need = (kv + ps - 1) // ps
    npg = int(need.sum()) + 7
    indptr = np.concatenate([[0], np.cumsum(need)]).astype(np.int32)
    indices = rng.permutation(npg)[:indptr[-1]].astype(np.int32)
    pool = random_pool(npg, 1, 4, ps, 128, device, 31)
    q, out, _ = run_decode(pool, 0, indptr, indices, kv, 8, device, 32)
    want = oracle_decode(pool, 0, indptr, indices, kv, q)
    assert max_abs(out, want) <= ATOL


def test_decode_empty_and_zero_length_rows(device):
    pool = random_pool(8, 1, 2, 16, 128, device, 41)
    indptr = np.array([0, 0, 1, 1], dtype=np.int32)
    indices = np.array([5], dtype=np.int32)
    kv = np.array([0, 9, 0], dtype=np.int32)
    q, out, _ = run_decode(pool, 0, indptr, indices, kv, 2, device, 42)
    want = oracle_decode(pool, 0, indptr, indices, kv, q)
    assert max_abs(out, want) <= ATOL
    assert torch.all(out[0] == 0) and torch.all(out[2] == 0)
    # no rows at all
    plan = DecodePlan(np.zeros(0, np.int32), 2, 2, device)
    assert plan.info.num_work == 0


def test_decode_split_invariance(device):
    """The result does not depend on the partition length (split-K + merge)."""
    rng = np.random.default_rng(5)
    kv = rng.integers(1, 9000, 24).astype(np.int32)
    need = (kv + 15) // 16
    indptr = np.concatenate([[0], np.cumsum(need)]).astype(np.int32)
    npg = int(indptr[-1]) + 5
    indices = rng.permutation(npg)[:indptr[-1]].astype(np.int32)
    pool = random_pool(npg, 1, 8, 16, 128, device, 51)
    outs = []
    for part in (256, 512, 2048, 4096):
        _, out, plan = run_decode(pool, 0, indptr, indices, kv, 32, device, 52, part)
        assert plan.info.part_tokens == part
        outs.append(out.float())
    for o in outs[1:]:
        assert max_abs(o, outs[0]) <= 1e-3
    q = random_tensor((len(kv), 32, 128), device, 52)
    rows = np.argsort(kv)[-4:]
    want = oracle_decode(pool, 0, indptr, indices, kv, q, rows)
    assert max_abs(outs[0][torch.from_numpy(rows).to(device)], want) <= ATOL


def test_decode_rows_of_more_than_64_partitions(device):
    """Rows split into more partitions than a wave has lanes (79 and 65 of
    256 tokens, and 8 and 9: one batch of partials and one more) merge in
    more than one round of log-sum-exps, and match the oracle and a plan
    with 4096-token partitions."""
    rng = np.random.default_rng(15)
    kv = np.array([20000, 17, 16400, 2048, 2049, 300], dtype=np.int32)
    need = (kv + 15) // 16
    indptr = np.concatenate([[0], np.cumsum(need)]).astype(np.int32)
    npg = int(indptr[-1]) + 3
    indices = rng.permutation(npg)[:indptr[-1]].astype(np.int32)
    pool = random_pool(npg, 1, 8, 16, 128, device, 53)
    q, out, plan = run_decode(pool, 0, indptr, indices, kv, 32, device, 54, 256)
    assert plan.info.part_tokens == 256 and plan.info.num_merge > 0
    want = oracle_decode(pool, 0, indptr, indices, kv, q)
    assert max_abs(out, want) <= ATOL
    _, out_long, _ = run_decode(pool, 0, indptr, indices, kv, 32, device, 54, 4096)
    assert max_abs(out, out_long.float()) <= 1e-3


def test_decode_page_permutation_bit_exact(device):
    """Moving pages (and the table with them) does not change one bit."""
    rng = np.random.default_rng(6)
    kv = np.array([40, 333, 1024], dtype=np.int32)
    need = (kv + 15) // 16
    indptr = np.concatenate([[0], np.cumsum(need)]).astype(np.int32)
    npg = 200
    indices = rng.permutation(npg)[:indptr[-1]].astype(np.int32)
    pool = random_pool(npg, 1, 4, 16, 128, device, 61)
    q, out, _ = run_decode(pool, 0, indptr, indices, kv, 4, device, 62)
    perm = rng.permutation(npg)
    pk, pv = torch.empty_like(pool.k), torch.empty_like(pool.v)
    idx = torch.from_numpy(perm).to(device)
    pk[idx], pv[idx] = pool.k, pool.v
    from kunserve_amd import KVPool
    moved = KVPool(pk, pv)
    _, out2, _ = run_decode(moved, 0, indptr, perm[indices].astype(np.int32), kv, 4, device, 62)
    assert torch.equal(out, out2)


def test_llama2_7b_decode_every_layer_and_row(device):
    """Full Llama-2-7B decode shape (32 layers, 16384-page pool, batch 64):
    every row of every layer against the fp32 reference on the device, and
    a sample of rows of three layers (the longest and the shortest among
    them) against the numpy oracle as well, which pins that reference at
    this shape."""
    w = workloads.llama2_7b_decode()
    pool = random_pool(w.num_pages, w.num_layers, w.num_kv_heads, w.page_size, w.head_dim,
                       device, 71)
    indptr, indices = w.csr()
    table = table_from_csr(indptr, indices, w.kv_len, device)
    plan = DecodePlan(w.kv_len, w.num_qo_heads, w.num_kv_heads, device)
    order = np.argsort(w.kv_len)
    rows = np.unique(np.concatenate([order[:2], order[-2:], order[::16]]))
    for layer in range(w.num_layers):
        q = random_tensor((w.batch, w.num_qo_heads, w.head_dim), device, 100 + layer)
        out = paged_decode(pool, layer, table, q, plan)
        full = torch_decode_ref(pool, layer, indptr, indices, w.kv_len, q)
        assert max_abs(out, full) <= ATOL, f"layer {layer}"
        if layer in (0, 13, 31):
            want = oracle_decode(pool, layer, indptr, indices, w.kv_len, q, rows)
            assert max_abs(out[torch.from_numpy(rows).to(device)], want) <= ATOL
            assert max_abs(full[torch.from_numpy(rows).to(device)], want) <= 1e-5


def test_llama3_8b_gqa_decode_every_row(device):
    """Llama-3-8B GQA decode (32 q / 8 KV heads, batch 128, contexts
    1024-8192, MFMA kernel with merges): every row against the fp32
    reference on the device, sampled rows against the numpy oracle."""
    w = workloads.llama3_8b_gqa_decode()
    pool = random_pool(w.num_pages, 1, w.num_kv_heads, w.page_size, w.head_dim, device, 81)
    indptr, indices = w.csr()
    q, out, plan = run_decode(pool, 0, indptr, indices, w.kv_len, w.num_qo_heads, device, 82)
    assert plan.info.num_merge > 0 and plan.info.group_size == 4
    assert max_abs(out, torch_decode_ref(pool, 0, indptr, indices, w.kv_len, q)) <= ATOL
    order = np.argsort(w.kv_len)
    rows = np.unique(np.concatenate([order[:2], order[-3:], order[::32]]))
    want = oracle_decode(pool, 0, indptr, indices, w.kv_len, q, rows)
    assert max_abs(out[torch.from_numpy(rows).to(device)], want) <= ATOL


def test_llama2_70b_decode_on_remapped_tables(device):
    """Block remap under memory pressure: copy 8192 random blocks between
    disjoint regions, then decode a Llama-2-70B layer (64 Q / 8 KV heads,
    batch 256, contexts U[256, 4096]) on tables pointing at the copies. The
    result equals the decode on the original tables bit for bit, the fp32
    reference on every row, and the oracle on sampled rows."""
    from kunserve_amd import copy_blocks

    r = workloads.kv_remap()
    pool = random_pool(r.num_pages, r.num_layers, r.num_kv_heads, r.page_size, r.head_dim,
                       device, 91)
    copy_blocks(pool, r.src, r.dst)
    w, w2 = r.decode, r.decode_remapped
    ip2, ix2 = w2.csr()
    q, out2, plan = run_decode(pool, 5, ip2, ix2, w2.kv_len, w2.num_qo_heads, device, 92)
    assert plan.info.group_size == 8
    ip, ix = w.csr()
    _, out, _ = run_decode(pool, 5, ip, ix, w.kv_len, w.num_qo_heads, device, 92)
    assert torch.equal(out.view(torch.int16), out2.view(torch.int16))
    assert max_abs(out2, torch_decode_ref(pool, 5, ip2, ix2, w2.kv_len, q)) <= ATOL
    order = np.argsort(w.kv_len)
    rows = np.unique(np.concatenate([order[:2], order[-2:], order[::64]]))
    want = oracle_decode(pool, 5, ip2, ix2, w2.kv_len, q, rows)
    assert max_abs(out2[torch.from_numpy(rows).to(device)], want) <= ATOL


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["f16", "bf16"])
@pytest.mark.parametrize("head_dim", [64, 128, 256])
@pytest.mark.parametrize("hq,hkv", [(8, 8), (8, 4)])
@pytest.mark.parametrize("num_cus", [3, 256])
def test_decode_plans_agree_with_each_other_and_the_oracle(device, dtype, head_dim, hq, hkv,
                                                           num_cus):
    """The automatic plan (long partitions when few CUs are assumed) and a
    fixed 512-token plan agree with the oracle and each other, in fp16 and
    bf16, with zero-length rows and rows from 1 to 9000 tokens."""
    rng = np.random.default_rng(head_dim + 10 * hq + hkv + num_cus)
    kv = np.array([0, 1, 5, 64, 65, 300, 1023, 4100, 9000, 17, 0, 2500], dtype=np.int32)
    need = (kv + 15) // 16
    indptr = np.concatenate([[0], np.cumsum(need)]).astype(np.int32)
    npg = int(indptr[-1]) + 3
    indices = rng.permutation(npg)[:indptr[-1]].astype(np.int32)
    pool = random_pool(npg, 1, hkv, 16, head_dim, device, 71, dtype=dtype)
    table = table_from_csr(indptr, indices, kv, device)
    q = random_tensor((len(kv), hq, head_dim), device, 72, dtype=dtype)
    auto = DecodePlan(kv, hq, hkv, device, num_cus=num_cus)
    fixed = DecodePlan(kv, hq, hkv, device, part_tokens=512, num_cus=num_cus)
    assert fixed.info.num_merge > 0
    out_a = paged_decode(pool, 0, table, q, auto).float()
    out_f = paged_decode(pool, 0, table, q, fixed).float()
    torch.cuda.synchronize()
    want = oracle_decode(pool, 0, indptr, indices, kv, q)
    tol = ATOL if dtype == torch.float16 else ATOL_BF16
    assert max_abs(out_a, want) <= tol
    assert max_abs(out_f, want) <= tol
    assert max_abs(out_a, out_f) <= tol
    assert torch.all(out_a[0] == 0) and torch.all(out_a[10] == 0)


def _small_decode_case(device, seed=81):
    rng = np.random.default_rng(seed)
    kv = rng.integers(1, 3000, 40).astype(np.int32)
    need = (kv + 15) // 16
    indptr = np.concatenate([[0], np.cumsum(need)]).astype(np.int32)
    npg = int(indptr[-1]) + 9
    indices = rng.permutation(npg)[:indptr[-1]].astype(np.int32)
    pool = random_pool(npg, 1, 8, 16, 128, device, seed)
    table = table_from_csr(indptr, indices, kv, device)
    q = random_tensor((len(kv), 8, 128), device, seed + 1)
    plan = DecodePlan(kv, 8, 8, device, part_tokens=256)
    return pool, table, q, plan, (indptr, indices, kv)


def test_decode_is_deterministic_over_many_launches_and_streams(device):
    """600 launches in a row, then launches on a second stream, give the
    bits of the first launch every time (no state carried between
    launches)."""
    pool, table, q, plan, (indptr, indices, kv) = _small_decode_case(device)
    ws = torch.empty(max(plan.workspace_bytes(128), 1), dtype=torch.uint8, device=device)
    first = paged_decode(pool, 0, table, q, plan, workspace=ws).clone()
    torch.cuda.synchronize()
    want = oracle_decode(pool, 0, indptr, indices, kv, q)
    assert max_abs(first, want) <= ATOL
    out = torch.empty_like(first)
    for i in range(600):
        paged_decode(pool, 0, table, q, plan, out=out, workspace=ws)
        if i % 100 == 99:
            torch.cuda.synchronize()
            assert torch.equal(out, first), f"launch {i}"
    s2 = torch.cuda.Stream(device)
    with torch.cuda.stream(s2):
        outs = [paged_decode(pool, 0, table, q, plan) for _ in range(4)]
    torch.cuda.synchronize()
    assert all(torch.equal(o, first) for o in outs)


def test_decode_graph_replays(device):
    """A decode launch captured in a HIP graph gives the eager result on
    every replay, with eager work and synchronisation between replays."""
    pool, table, q, plan, _ = _small_decode_case(device, 91)
    ws = torch.empty(max(plan.workspace_bytes(128), 1), dtype=torch.uint8, device=device)
    out = torch.empty_like(q)
    eager = paged_decode(pool, 0, table, q, plan, workspace=ws).clone()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        paged_decode(pool, 0, table, q, plan, out=out, workspace=ws)
    for r in range(5):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {r}"
        paged_decode(pool, 0, table, q, plan, workspace=ws)   # eager launch between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("ratio", [4, 8])
def test_gqa_decode_equals_mha_on_repeated_heads(device, ratio):
    """GQA decode (the MFMA kernel for 4 and 8 q heads per KV head) equals
    MHA decode (the VALU kernel) on a pool whose KV heads are repeated
    `ratio` times, each q head reading its own copy."""
    from kunserve_amd import KVPool
    rng = np.random.default_rng(ratio)
    hkv, hq = 4, 4 * ratio
    kv = np.array([1, 33, 700, 2049, 5000, 16], dtype=np.int32)
    need = (kv + 15) // 16
    indptr = np.concatenate([[0], np.cumsum(need)]).astype(np.int32)
    npg = int(indptr[-1]) + 4
    indices = rng.permutation(npg)[:indptr[-1]].astype(np.int32)
    pool = random_pool(npg, 1, hkv, 16, 128, device, 111)
    mha = KVPool(pool.k.repeat_interleave(ratio, dim=2).contiguous(),
                 pool.v.repeat_interleave(ratio, dim=2).contiguous())
    table = table_from_csr(indptr, indices, kv, device)
    q = random_tensor((len(kv), hq, 128), device, 112)
    gqa_plan = DecodePlan(kv, hq, hkv, device)
    mha_plan = DecodePlan(kv, hq, hq, device)
    assert gqa_plan.info.group_size == min(ratio, 8) and mha_plan.info.group_size == 1
    out_g = paged_decode(pool, 0, table, q, gqa_plan).float()
    out_m = paged_decode(mha, 0, table, q, mha_plan).float()
    torch.cuda.synchronize()
    assert max_abs(out_g, out_m) <= ATOL


@pytest.mark.parametrize("hq,hkv", [(8, 8), (32, 4)])
def test_decode_closed_forms(device, hq, hkv):
    """One cached token gives its V row exactly; q = 0 gives the mean of the
    row's V (uniform weights), on the VALU (G = 1) and MFMA (G = 8) kernels."""
    rng = np.random.default_rng(hq + hkv)
    kv = np.array([1, 1, 300, 4097], dtype=np.int32)
    need = (kv + 15) // 16
    indptr = np.concatenate([[0], np.cumsum(need)]).astype(np.int32)
    npg = int(indptr[-1]) + 2
    indices = rng.permutation(npg)[:indptr[-1]].astype(np.int32)
    pool = random_pool(npg, 1, hkv, 16, 128, device, 121)
    table = table_from_csr(indptr, indices, kv, device)
    plan = DecodePlan(kv, hq, hkv, device, part_tokens=1024)
    q = random_tensor((len(kv), hq, 128), device, 122)
    q[2:] = 0
    out = paged_decode(pool, 0, table, q, plan)
    torch.cuda.synchronize()
    ratio = hq // hkv
    for b in (0, 1):
        v0 = pool.v[int(indices[indptr[b]]), 0, :, 0]            # [hkv, D]
        assert torch.equal(out[b], v0.repeat_interleave(ratio, dim=0))
    for b in (2, 3):
        pages = torch.from_numpy(indices[indptr[b]:indptr[b + 1]].astype(np.int64)).to(device)
        rows = pool.v[pages, 0].permute(1, 0, 2, 3).reshape(hkv, -1, 128)[:, :int(kv[b])]
        mean = rows.float().mean(dim=1).repeat_interleave(ratio, dim=0)
        assert max_abs(out[b].float(), mean) <= ATOL
