"""bf16 pools (the reference's default --dtype, kunserve/kunserve_config.py:61)
on the GPU vs the CPU oracle evaluated on the same bf16 values.

Attention: max-abs <= ATOL_BF16 (bf16 keeps 8 significant bits to fp16's 11)
and relative Frobenius error <= RTOL_BF16.
RoPE: one bf16 ulp plus 1e-6. Block movement: bit-exact (byte copies)."""
import math

import numpy as np
import pytest
import torch

from kunserve_amd import (AttentionStep, DecodePlan, LlamaOp, PrefillPlan, append_kv,
                          copy_blocks, paged_decode, paged_prefill, rope_append_kv,
                          rope_inv_freq)
from oracle import paged_attention_ref as ref

from helpers import (ATOL_BF16, RTOL_BF16, compact_for_oracle, max_abs, random_pool,
                     random_tensor, rel_err, table_from_csr, to_numpy)

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


def rows_csr(rng, kv, ps, npg):
    kv = np.asarray(kv, dtype=np.int32)
    need = (kv + ps - 1) // ps
    indptr = np.concatenate([[0], np.cumsum(need)]).astype(np.int32)
    indices = rng.permutation(npg)[:indptr[-1]].astype(np.int32)
    return kv, indptr, indices


@pytest.mark.parametrize("head_dim", [64, 128, 256])
@pytest.mark.parametrize("hq,hkv", [(8, 8), (8, 2), (32, 8), (16, 2)])
def test_bf16_decode_matches_oracle(device, head_dim, hq, hkv):
    """Group 1 and 2 run the VALU kernel; 4 and 8 at head_dim 128 the MFMA one."""
    rng = np.random.default_rng(head_dim + hq)
    kv, indptr, indices = rows_csr(rng, [1, 15, 16, 17, 300, 1000, 2500], 16, 400)
    pool = random_pool(400, 1, hkv, 16, head_dim, device, 1, dtype=BF16)
    q = random_tensor((len(kv), hq, head_dim), device, 2, dtype=BF16)
    out = paged_decode(pool, 0, table_from_csr(indptr, indices, kv, device), q,
                       DecodePlan(kv, hq, hkv, device, part_tokens=256))
    torch.cuda.synchronize()
    assert out.dtype == BF16
    k, v, ip, ix = compact_for_oracle(pool, 0, indptr, indices)
    want = ref.decode_attention(to_numpy(q), k, v, 0, ip, ix, kv, 1 / math.sqrt(head_dim))
    assert max_abs(out, want) <= ATOL_BF16
    assert rel_err(out, want) <= RTOL_BF16, rel_err(out, want)


@pytest.mark.parametrize("num_cus", [1, 1024])
@pytest.mark.parametrize("head_dim", [64, 128, 256])
def test_bf16_prefill_matches_oracle(device, num_cus, head_dim):
    """Whole KV ranges (num_cus 1) and split ones (num_cus 1024), head_dim
    64, 128 and 256."""
    rng = np.random.default_rng(num_cus)
    q_lens, prefixes = [1, 77, 256, 300, 512], [700, 0, 1500, 33, 2048]
    kv = np.asarray(q_lens) + np.asarray(prefixes)
    kv, indptr, indices = rows_csr(rng, kv, 16, 600)
    q_indptr = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    pool = random_pool(600, 1, 4, 16, head_dim, device, 3, dtype=BF16)
    q = random_tensor((int(q_indptr[-1]), 8, head_dim), device, 4, dtype=BF16)
    plan = PrefillPlan(q_indptr, kv, 8, 4, device, num_cus=num_cus, head_dim=head_dim)
    assert (plan.info.num_merge > 0) == (num_cus == 1024)
    out = paged_prefill(pool, 0, table_from_csr(indptr, indices, kv, device),
                        torch.from_numpy(q_indptr).to(device), q, plan)
    torch.cuda.synchronize()
    k, v, ip, ix = compact_for_oracle(pool, 0, indptr, indices)
    want = ref.prefill_attention(to_numpy(q), q_indptr, k, v, 0, ip, ix, kv,
                                 1 / math.sqrt(head_dim))
    assert max_abs(out, want) <= ATOL_BF16
    assert rel_err(out, want) <= RTOL_BF16, rel_err(out, want)


def test_bf16_rope_append_and_block_moves(device):
    rng = np.random.default_rng(5)
    q_lens, prefixes = [3, 1, 70], [0, 500, 10]
    kv = np.asarray(q_lens) + np.asarray(prefixes)
    kv, indptr, indices = rows_csr(rng, kv, 16, 80)
    q_indptr = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    T = int(q_indptr[-1])
    pool = random_pool(80, 2, 2, 16, 128, device, 6, dtype=BF16)
    k0, v0 = to_numpy(pool.k), to_numpy(pool.v)
    q = random_tensor((T, 4, 128), device, 7, dtype=BF16)
    kn, vn = (random_tensor((T, 2, 128), device, s, dtype=BF16) for s in (8, 9))
    q_in, kn_in, vn_in = to_numpy(q), to_numpy(kn), to_numpy(vn)
    inv = rope_inv_freq(128, 10000.0, device)
    table = table_from_csr(indptr, indices, kv, device)
    rope_append_kv(pool, 1, table, torch.from_numpy(q_indptr).to(device), q, kn, vn, inv)
    torch.cuda.synchronize()
    pos = ref.token_positions(kv, q_indptr)
    want_q = ref.rope(q_in, pos, inv.cpu().numpy(), False)
    want_q16 = torch.from_numpy(want_q).to(BF16).float().numpy()
    ulp = np.abs(want_q16) * 2.0 ** -7 + 1e-6
    assert np.all(np.abs(to_numpy(q) - want_q16) <= ulp)
    # v lands bit-exactly; then a block copy moves the bf16 bits unchanged
    ve = v0.copy()
    ref.append_kv(np.zeros_like(k0), ve, 1, indptr, indices, kv, q_indptr, kn_in, vn_in)
    assert np.array_equal(to_numpy(pool.v), ve)
    free = [p for p in range(80) if p not in set(indices.tolist())]
    src, dst = [int(indices[0]), int(indices[1])], free[:2]
    before = to_numpy(pool.k)
    copy_blocks(pool, src, dst)
    torch.cuda.synchronize()
    after = to_numpy(pool.k)
    assert np.array_equal(after[dst], before[src])


def test_bf16_llama_op_mixed_step(device):
    """LlamaOp with a bf16 pool: one decode row and one chunked-prefill row."""
    op = LlamaOp(64, 2, 8, 2, 16, 128, 11008, 32000, 8, 4096, 4096, 1, device=device,
                 dtype=BF16)
    g = torch.Generator(device=device)
    g.manual_seed(10)
    for t in (op.pool.k, op.pool.v):
        t.copy_(torch.randn(t.shape, generator=g, device=device).to(BF16))
    q_lens, first, flags = [1, 33], [40, 7], [0, 1]
    pages = [list(range(0, 3)), list(range(10, 13))]
    step = op.pforward(2, 34, 64, 0, 2, [[0] * n for n in q_lens], first, flags, pages)
    q = random_tensor((34, 8, 128), device, 11, dtype=BF16)
    k, v = (random_tensor((34, 2, 128), device, s, dtype=BF16) for s in (12, 13))
    k_pool0, v_pool0 = to_numpy(op.pool.k), to_numpy(op.pool.v)
    out = step.run(1, q, k, v)
    torch.cuda.synchronize()
    kv = np.array([40, 40], dtype=np.int64)   # decode: first; prefill: first + q_len
    q_indptr = np.array([0, 1, 34])
    indptr = np.array([0, 3, 6])
    indices = np.array(pages[0] + pages[1])
    ref.append_kv(k_pool0, v_pool0, 1, indptr, indices, kv, q_indptr, to_numpy(k), to_numpy(v))
    want = ref.prefill_attention(to_numpy(q), q_indptr, k_pool0, v_pool0, 1, indptr, indices, kv,
                                 1 / math.sqrt(128))
    assert out.dtype == BF16 and max_abs(out, want) <= ATOL_BF16
    assert rel_err(out, want) <= RTOL_BF16, rel_err(out, want)


def test_bf16_decode_on_256_token_pages(device):
    """The reference's default configuration: bf16 pool, 256-token pages,
    rows that end inside a page and rows longer than one partition."""
    rng = np.random.default_rng(256)
    kv = np.array([1, 255, 256, 257, 3000, 9000], dtype=np.int32)
    need = (kv + 255) // 256
    indptr = np.concatenate([[0], np.cumsum(need)]).astype(np.int32)
    npg = int(indptr[-1]) + 3
    indices = rng.permutation(npg)[:indptr[-1]].astype(np.int32)
    pool = random_pool(npg, 1, 8, 256, 128, device, 257, dtype=BF16)
    table = table_from_csr(indptr, indices, kv, device)
    q = random_tensor((len(kv), 8, 128), device, 258, dtype=BF16)
    plan = DecodePlan(kv, 8, 8, device, part_tokens=512)
    out = paged_decode(pool, 0, table, q, plan)
    torch.cuda.synchronize()
    k, v, ip, ix = compact_for_oracle(pool, 0, indptr, indices, np.arange(len(kv)))
    want = ref.decode_attention(to_numpy(q), k, v, 0, ip, ix, kv, 1.0 / math.sqrt(128))
    assert max_abs(out, want) <= ATOL_BF16
    assert rel_err(out, want) <= RTOL_BF16, rel_err(out, want)
