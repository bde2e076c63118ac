"""Shared helpers for the parity tests (tables, inputs, closed forms)."""
from __future__ import annotations

import numpy as np

MICRO, EXTENT = 0, 1

DESC = np.dtype({
    "names": ["slot", "generation", "logical_token_begin", "valid_tokens", "page_token_capacity", "kind"],
    "formats": ["<u4", "<u4", "<u4", "<u2", "<u2", "u1"],
    "offsets": [0, 4, 8, 12, 14, 16],
    "itemsize": 20,
})


def splitmix_permutation(seed: int, n: int) -> np.ndarray:
    """Fisher-Yates driven by splitmix64 (same sequence as kimkv_seeded_permutation)."""
    mask = (1 << 64) - 1
    out = list(range(n))
    state = seed & mask
    for i in range(n, 1, -1):
        state = (state + 0x9E3779B97F4A7C15) & mask
        z = state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask
        z ^= z >> 31
        j = z % i
        out[i - 1], out[j] = out[j], out[i - 1]
    return np.array(out, dtype=np.uint32)


class SlotAllocator:
    """Hands out slots of each pool in a seeded permuted order."""

    def __init__(self, micro_capacity: int, extent_capacity: int, seed: int = 7,
                 micro_tokens: int = 8, extent_tokens: int = 64):
        self.free = {MICRO: list(splitmix_permutation(seed, micro_capacity)),
                     EXTENT: list(splitmix_permutation(seed + 1, extent_capacity))}
        self.cap = {MICRO: micro_tokens, EXTENT: extent_tokens}

    def take(self, kind: int) -> int:
        return int(self.free[kind].pop(0))


def hetero_table(tokens: int, alloc: SlotAllocator) -> np.ndarray:
    """Block table with floor(T/64) extents then ceil((T%64)/8) micro pages
    (the layout repeated append-64 + promote produces)."""
    entries = []
    begin = 0
    et, mt = alloc.cap[EXTENT], alloc.cap[MICRO]
    while tokens - begin >= et:
        entries.append((alloc.take(EXTENT), 1, begin, et, et, EXTENT))
        begin += et
    while begin < tokens:
        n = min(mt, tokens - begin)
        entries.append((alloc.take(MICRO), 1, begin, n, mt, MICRO))
        begin += n
    return np.array(entries, dtype=DESC)


def uniform_table(tokens: int, page_tokens: int, alloc: SlotAllocator, kind: int = MICRO) -> np.ndarray:
    entries = []
    begin = 0
    while begin < tokens:
        n = min(page_tokens, tokens - begin)
        entries.append((alloc.take(kind), 1, begin, n, page_tokens, kind))
        begin += n
    return np.array(entries, dtype=DESC)


def entries_to_desc(entries, micro_tokens: int = 8, extent_tokens: int = 64) -> np.ndarray:
    """Mapping entries (begin, valid, kind, slot, generation) -> descriptor array."""
    out = np.zeros(len(entries), dtype=DESC)
    for i, (begin, valid, kind, slot, gen) in enumerate(entries):
        out[i] = (slot, gen, begin, valid, micro_tokens if kind == MICRO else extent_tokens, kind)
    return out


def make_kv_closed_form(layers: int, heads: int, dim: int, begin: int, count: int) -> np.ndarray:
    """The reference's makeKv generator (tests/cuda/cuda_kv_test.cpp:127-172):
    0.125*layer + 0.25*comp + token/128 + head/32 + dim/256 - 0.5, every value
    exact in fp16.  Returns [L][2][count][H][D] as float16 codes."""
    l = np.arange(layers, dtype=np.float64)[:, None, None, None, None]
    c = np.arange(2, dtype=np.float64)[None, :, None, None, None]
    t = (begin + np.arange(count, dtype=np.float64))[None, None, :, None, None]
    h = np.arange(heads, dtype=np.float64)[None, None, None, :, None]
    d = np.arange(dim, dtype=np.float64)[None, None, None, None, :]
    v = 0.125 * l + 0.25 * c + 0.0078125 * t + 0.03125 * h + 0.00390625 * d - 0.5
    return v.astype(np.float16).view(np.uint16)


def to_f32(codes: np.ndarray) -> np.ndarray:
    return np.asarray(codes, dtype=np.uint16).view(np.float16).astype(np.float32)


def assert_attention_close(actual_codes: np.ndarray, expected_f32: np.ndarray, atol=2e-3, rtol=1e-3):
    """Decode tolerance: |gpu - ref| <= 2e-3 + 1e-3 * |ref| against the fp32-accumulated oracle."""
    actual = to_f32(actual_codes)
    expected = np.asarray(expected_f32, dtype=np.float32)
    err = np.abs(actual - expected)
    bound = atol + rtol * np.abs(expected)
    bad = np.nonzero(err > bound)[0]
    assert bad.size == 0, (
        f"{bad.size} of {err.size} outputs out of tolerance; worst at {bad[np.argmax(err[bad] - bound[bad])]} "
        f"err={err.max():.3e}")
    return float(err.max())
