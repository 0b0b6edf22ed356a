"""The committed golden vectors (tests/golden/*.npz) still follow from the
CPU oracle: guards the oracle against drift (CPU only)."""
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import paged_attention_ref as ref

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_decode_golden():
    g = load("decode")
    out = ref.decode_attention(g["q"], g["k"], g["v"], int(g["layer"]), g["indptr"], g["indices"],
                               g["kv_len"], 1 / math.sqrt(g["q"].shape[-1]))
    np.testing.assert_allclose(out, g["out"], rtol=0, atol=1e-6)
    assert np.all(g["out"][g["kv_len"] == 0] == 0)


def test_prefill_golden():
    g = load("prefill")
    out = ref.prefill_attention(g["q"], g["q_indptr"], g["k"], g["v"], 0, g["indptr"],
                                g["indices"], g["kv_len"], 1 / math.sqrt(g["q"].shape[-1]))
    np.testing.assert_allclose(out, g["out"], rtol=0, atol=1e-6)


def test_append_golden():
    g = load("append")
    k, v = g["k"].copy(), g["v"].copy()
    ref.append_kv(k, v, int(g["layer"]), g["indptr"], g["indices"], g["kv_len"], g["q_indptr"],
                  g["k_new"], g["v_new"])
    assert np.array_equal(k.view(np.int16), g["k_out"].view(np.int16))
    assert np.array_equal(v.view(np.int16), g["v_out"].view(np.int16))


def test_copy_golden():
    g = load("copy")
    k = g["k"].copy()
    ref.copy_blocks(k, g["src"], g["dst"])
    assert np.array_equal(k, g["k_out"])
    assert np.array_equal(ref.kv_pack(g["k"], g["v"], 1, 3, g["src"]), g["pack_scratch"])
