"""Seeded paged-KV-cache builders — TEST INFRASTRUCTURE.

Mirror the reference tests' builders (tests/test_paged_attention.py:10-73,
tests/test_paged_long_context.py:11-36): contiguous [B, Hkv, T, D] K/V are cut
into pages of ``page_size`` tokens, placed at physical page indices given by a
sequential or a shuffled (seeded ``randperm``) assignment, and described by an
int32 block table [B, max_pages] plus int32 context lengths [B].
Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py`` use this module.
"""
from __future__ import annotations

import torch


def build_paged_cache(k, v, page_size=16, *, shuffle=False, generator=None, context_lens=None):
    """Return (k_cache, v_cache, block_table, context_lens) on the CPU.

    ``context_lens`` (optional, list of ints <= T) gives per-sequence lengths;
    pages past a sequence's length stay zero, as in
    tests/test_paged_attention.py:181-206.
    """
    B, Hkv, T, D = k.shape
    per_seq = (T + page_size - 1) // page_size
    total = B * per_seq
    k_cache = torch.zeros(total, Hkv, page_size, D, dtype=k.dtype)
    v_cache = torch.zeros(total, Hkv, page_size, D, dtype=v.dtype)
    table = torch.zeros(B, per_seq, dtype=torch.int32)
    lens = [T] * B if context_lens is None else list(context_lens)
    if shuffle:
        perm = torch.randperm(total, generator=generator)
    else:
        perm = torch.arange(total)
    for b in range(B):
        for blk in range(per_seq):
            phys = int(perm[b * per_seq + blk])
            table[b, blk] = phys
            start = blk * page_size
            end = min(start + page_size, lens[b])
            if end > start:
                k_cache[phys, :, : end - start] = k[b, :, start:end]
                v_cache[phys, :, : end - start] = v[b, :, start:end]
    return k_cache, v_cache, table, torch.tensor(lens, dtype=torch.int32)


def random_paged_layout(context_lens, page_size, *, generator):
    """Block table for a serving-style cache: a seeded permutation of all
    physical pages, assigned to sequences in order; unused entries are 0.

    Returns (block_table int32 [B, max_pages], n_pages).  Used for the decode
    benchmark, where K/V pages are drawn directly (no contiguous source).
    """
    npg = [(int(c) + page_size - 1) // page_size for c in context_lens]
    total = sum(npg)
    perm = torch.randperm(total, generator=generator).to(torch.int32)
    table = torch.zeros(len(npg), max(npg), dtype=torch.int32)
    pos = 0
    for b, n in enumerate(npg):
        table[b, :n] = perm[pos:pos + n]
        pos += n
    return table, total


def append_kv(k_cache, v_cache, k_new, v_new, block_table, context_lens):
    """Reference semantics of the paged-KV append, element by element on the
    CPU (the reference fills caches with the same index arithmetic in its
    test builders, tests/test_paged_attention.py:10-73): row t of sequence b
    goes to page block_table[b, (ctx_b + t) // P], slot (ctx_b + t) % P;
    rows whose page index is past the table or whose entry is outside the
    cache are dropped.  Returns new (k_cache, v_cache) copies.

    pinned by: appending a whole sequence into an empty cache reproduces
    build_paged_cache, and appends in pieces equal one append.
    """
    kc, vc = k_cache.clone(), v_cache.clone()
    n_pages, _, P, _ = kc.shape
    B, H, n_new, _ = k_new.shape
    for b in range(B):
        for t in range(n_new):
            pos = int(context_lens[b]) + t
            pi = pos // P
            if pi >= block_table.shape[1]:
                continue
            phys = int(block_table[b, pi])
            if phys < 0 or phys >= n_pages:
                continue
            kc[phys, :, pos % P] = k_new[b, :, t]
            vc[phys, :, pos % P] = v_new[b, :, t]
    return kc, vc
