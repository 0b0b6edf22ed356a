"""HIP kernels against the committed golden vectors (tests/golden/*.npz)."""
from pathlib import Path

import numpy as np
import pytest
import torch

from kunserve_amd import (DecodePlan, KVPool, PrefillPlan, append_kv, copy_blocks, kv_pack,
                          paged_decode, paged_prefill)

from helpers import ATOL, max_abs, table_from_csr

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def pool_of(g, device, kk="k", vk="v"):
    k = torch.from_numpy(g[kk]).to(device)
    v = torch.from_numpy(g[vk]).to(device)
    if k.dtype == torch.int16:
        k, v = k.view(torch.float16), v.view(torch.float16)
    return KVPool(k, v)


def test_decode_golden(device):
    g = load("decode")
    pool = pool_of(g, device)
    table = table_from_csr(g["indptr"], g["indices"], g["kv_len"], device)
    q = torch.from_numpy(g["q"]).to(device)
    plan = DecodePlan(g["kv_len"], q.shape[1], pool.num_kv_heads, device)
    out = paged_decode(pool, int(g["layer"]), table, q, plan)
    assert max_abs(out, g["out"]) <= ATOL


def test_prefill_golden(device):
    g = load("prefill")
    pool = pool_of(g, device)
    table = table_from_csr(g["indptr"], g["indices"], g["kv_len"], device)
    q = torch.from_numpy(g["q"]).to(device)
    plan = PrefillPlan(g["q_indptr"], g["kv_len"], q.shape[1], pool.num_kv_heads, device)
    out = paged_prefill(pool, 0, table, torch.from_numpy(g["q_indptr"]).to(device), q, plan)
    assert max_abs(out, g["out"]) <= ATOL


def test_append_golden(device):
    g = load("append")
    pool = pool_of(g, device)
    table = table_from_csr(g["indptr"], g["indices"], g["kv_len"], device)
    append_kv(pool, int(g["layer"]), table, torch.from_numpy(g["q_indptr"]).to(device),
              torch.from_numpy(g["k_new"]).to(device), torch.from_numpy(g["v_new"]).to(device))
    torch.cuda.synchronize()
    assert np.array_equal(pool.k.cpu().numpy().view(np.int16), g["k_out"].view(np.int16))
    assert np.array_equal(pool.v.cpu().numpy().view(np.int16), g["v_out"].view(np.int16))


def test_copy_and_pack_golden(device):
    g = load("copy")
    pool = pool_of(g, device)
    scratch = kv_pack(pool, 1, 3, g["src"].tolist())
    copy_blocks(pool, g["src"].tolist(), g["dst"].tolist())
    torch.cuda.synchronize()
    assert np.array_equal(pool.k.view(torch.int16).cpu().numpy(), g["k_out"])
    assert np.array_equal(pool.v.view(torch.int16).cpu().numpy(), g["v_out"])
    want = g["pack_scratch"]
    got = scratch.view(torch.int16).cpu().numpy()[:want.size].reshape(want.shape)
    assert np.array_equal(got, want)
