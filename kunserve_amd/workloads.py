"""Seeded synthetic workloads at the named serving shapes (host side, numpy).

Each generator returns page tables and lengths only; tensors are filled on
the device by the caller. Seeds are fixed per workload so that every run
(tests, bench) draws the same lengths and tables.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np


@dataclass
class DecodeShape:
    name: str
    num_layers: int           # layers of the KV pool
    num_qo_heads: int
    num_kv_heads: int
    head_dim: int
    page_size: int
    num_pages: int
    kv_len: np.ndarray        # [B] int32
    pages: list               # B arrays of page ids (ceil(kv_len / page_size) each)
    seed: int

    @property
    def batch(self) -> int:
        return len(self.kv_len)

    def csr(self) -> tuple[np.ndarray, np.ndarray]:
        indptr = np.zeros(self.batch + 1, dtype=np.int32)
        np.cumsum([len(p) for p in self.pages], out=indptr[1:])
        indices = (np.concatenate(self.pages).astype(np.int32) if self.pages
                   else np.zeros(0, np.int32))
        return indptr, indices

    def kv_bytes_per_layer(self) -> int:
        """Algorithmic HBM bytes of one decode launch: K and V of every cached
        token of every KV head once, q and out once, the page ids once."""
        tok = int(self.kv_len.astype(np.int64).sum())
        kv = tok * self.num_kv_heads * self.head_dim * 2 * 2
        qo = 2 * self.batch * self.num_qo_heads * self.head_dim * 2
        tbl = sum(len(p) for p in self.pages) * 4
        return kv + qo + tbl


def _tables(rng: np.random.Generator, kv_len: np.ndarray, page_size: int, num_pages: int,
            exclude: Optional[np.ndarray] = None) -> list:
    """Disjoint random page lists drawn from a permutation of the pool."""
    perm = rng.permutation(num_pages)
    if exclude is not None:
        perm = perm[~np.isin(perm, exclude)]
    need = (kv_len.astype(np.int64) + page_size - 1) // page_size
    if need.sum() > perm.size:
        raise ValueError(f"{int(need.sum())} pages needed, pool offers {perm.size}")
    out, at = [], 0
    for n in need:
        out.append(perm[at:at + n].astype(np.int32))
        at += int(n)
    return out


def single_layer_decode(seed: int = 1001) -> DecodeShape:
    """1 layer, fp16, batch 8, 32 Q = 32 KV heads, head_dim 128, page 16,
    contexts U[128, 512], tables from a permutation of a 512-page pool."""
    rng = np.random.default_rng(seed)
    kv = rng.integers(128, 513, size=8).astype(np.int32)
    return DecodeShape("single-layer decode b8 h32 ctx128-512", 1, 32, 32, 128, 16, 512, kv,
                       _tables(rng, kv, 16, 512), seed)


def llama2_7b_decode(seed: int = 1002, page_size: int = 16) -> DecodeShape:
    """Llama-2-7B decode: 32 layers, 32/32 heads, head_dim 128, a pool of
    262144 tokens (16384 pages of 16, or 1024 of 256: the reference's
    default block size), batch 64, contexts round(lognormal(ln 700, 1.0))
    clipped to [16, 4096]."""
    rng = np.random.default_rng(seed)
    kv = np.clip(np.round(rng.lognormal(np.log(700.0), 1.0, size=64)), 16, 4096).astype(np.int32)
    num_pages = 16384 * 16 // page_size
    name = "llama2-7b decode b64 ctx lognormal(700) x32 layers"
    if page_size != 16:
        name += f" page{page_size}"
    return DecodeShape(name, 32, 32, 32, 128, page_size, num_pages, kv,
                       _tables(rng, kv, page_size, num_pages), seed)


def llama3_8b_gqa_decode(seed: int = 1003) -> DecodeShape:
    """Llama-3-8B GQA decode: 32 Q / 8 KV heads, head_dim 128, page 16,
    batch 128, contexts U[1024, 8192], one layer."""
    rng = np.random.default_rng(seed)
    kv = rng.integers(1024, 8193, size=128).astype(np.int32)
    pool = 40960
    return DecodeShape("llama3-8b gqa decode b128 ctx1024-8192", 1, 32, 8, 128, 16, pool, kv,
                       _tables(rng, kv, 16, pool), seed)


@dataclass
class PrefillShape:
    name: str
    num_qo_heads: int
    num_kv_heads: int
    head_dim: int
    page_size: int
    num_pages: int
    prompt_len: np.ndarray    # [S]
    prefix_len: np.ndarray    # [S] tokens already in pages before the prompt
    chunk: int
    pages: list               # S arrays: pages for prefix + prompt
    seed: int

    def steps(self) -> list:
        """Chunked-prefill steps: each step takes the next <= chunk tokens of
        every unfinished sequence (kunserve/request.py:368-391). Returns a list
        of (rows, q_len, kv_len_after) triples of int arrays."""
        done = np.zeros_like(self.prompt_len)
        out = []
        while np.any(done < self.prompt_len):
            rows = np.nonzero(done < self.prompt_len)[0]
            ql = np.minimum(self.chunk, self.prompt_len[rows] - done[rows])
            kv_after = self.prefix_len[rows] + done[rows] + ql
            out.append((rows, ql.astype(np.int32), kv_after.astype(np.int32)))
            done[rows] += ql
        return out

    def causal_flops(self) -> int:
        """Exact causal flops of all steps: 4 * Hq * D per (query, visible key)."""
        total = 0
        for _, ql, kv in self.steps():
            for q, k in zip(ql.tolist(), kv.tolist()):
                first = k - q
                # sum over i in [0, q) of (first + i + 1)
                total += q * first + q * (q + 1) // 2
        return 4 * self.num_qo_heads * self.head_dim * total


def chunked_prefill(seed: int = 1004, num_pages: int | None = None,
                    page_size: int = 16) -> PrefillShape:
    """16 sequences, prompts U[512, 4096], prefixes U[0, 2048] already in
    pages, chunk 512, Llama-2-7B heads (32/32, head_dim 128), page 16 (or
    page_size; the pool holds the same 131072 tokens by default)."""
    rng = np.random.default_rng(seed)
    prompt = rng.integers(512, 4097, size=16).astype(np.int32)
    prefix = rng.integers(0, 2049, size=16).astype(np.int32)
    if num_pages is None:
        num_pages = 8192 * 16 // page_size
    pages = _tables(rng, prompt + prefix, page_size, num_pages)
    name = "chunked prefill 16 seqs prompt512-4096 prefix0-2048 chunk512"
    if page_size != 16:
        name += f" page{page_size}"
    return PrefillShape(name, 32, 32, 128, page_size, num_pages, prompt, prefix, 512, pages, seed)


@dataclass
class RemapShape:
    """Block remap under memory pressure: copy n_copy blocks from region
    [0, n_copy) to region [n_copy, 2 n_copy), then decode on tables whose
    copied pages point at the copies."""
    num_pages: int
    num_layers: int
    num_kv_heads: int
    page_size: int
    head_dim: int
    src: np.ndarray
    dst: np.ndarray
    decode: DecodeShape
    decode_remapped: DecodeShape = field(repr=False, default=None)
    seed: int = 1005

    def copy_bytes(self) -> int:
        """Read + write bytes of the copy (K and V, all layers)."""
        block = self.num_layers * self.num_kv_heads * self.page_size * self.head_dim * 2
        return 2 * 2 * block * len(self.src)


def kv_remap(seed: int = 1005, n_copy: int = 8192, num_pages: int = 45056,
             batch: int = 256) -> RemapShape:
    """8192 random blocks of [32 layers, 8 heads, 16, 128] fp16 copied between
    disjoint regions; then a Llama-2-70B layer decode (64 Q / 8 KV heads,
    batch 256, contexts U[256, 4096]) whose tables point at the copies."""
    rng = np.random.default_rng(seed)
    src = rng.permutation(n_copy).astype(np.int32)
    dst = (n_copy + rng.permutation(n_copy)).astype(np.int32)
    kv = rng.integers(256, 4097, size=batch).astype(np.int32)
    # Tables never use the destination region, so every copied page is
    # reachable only through the remap below.
    tables = _tables(rng, kv, 16, num_pages, exclude=np.arange(n_copy, 2 * n_copy))
    dec = DecodeShape("llama2-70b layer decode b256 ctx256-4096", 32, 64, 8, 128, 16, num_pages,
                      kv, tables, seed)
    remap = np.arange(num_pages, dtype=np.int32)
    remap[src] = dst
    dec2 = DecodeShape(dec.name + " (remapped tables)", 32, 64, 8, 128, 16, num_pages, kv,
                       [remap[p] for p in tables], seed)
    return RemapShape(num_pages, 32, 8, 16, 128, src, dst, dec, dec2, seed)
