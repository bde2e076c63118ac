"""Pins the CPU oracle before anything is compared against it.

Each check is independent of the oracle's own code: the reference's
known-answer vectors, numpy's float16 conversion (a library routine), the
reference's own CPU library built in oracle/_ref, closed forms, and brute force
in float64.
"""
import ctypes
import math

import numpy as np
import pytest

import oracle
from tests import helpers


# ---- fp16 codec -------------------------------------------------------------

def test_codec_known_answers():
    # tests/reference/kv_reference_test.cpp:24-43
    enc = oracle.lib().kvo_f32_to_f16
    dec = oracle.lib().kvo_f16_to_f32
    assert enc(0.0) == 0x0000
    assert enc(-0.0) == 0x8000
    assert enc(1.0) == 0x3C00
    assert enc(-2.0) == 0xC000
    assert enc(65504.0) == 0x7BFF
    assert dec(0x3C00) == 1.0
    assert dec(0xC000) == -2.0
    assert dec(0x7BFF) == 65504.0
    assert math.isinf(dec(0x7C00))
    assert math.isnan(dec(0x7E00))


def test_decode_all_codes_match_numpy():
    codes = np.arange(65536, dtype=np.uint16)
    ours = oracle.f16_to_f32(codes)
    ref = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_encode_matches_numpy_rne():
    rng = np.random.default_rng(1)
    parts = [
        rng.standard_normal(200000).astype(np.float32) * 4,
        (rng.standard_normal(50000) * 1e-5).astype(np.float32),      # subnormal range
        (rng.standard_normal(50000) * 7e4).astype(np.float32),       # overflow range
        np.array([65519.0, 65520.0, 2.0 ** -25, 2.0 ** -24, 3 * 2.0 ** -26, -0.0, np.inf, -np.inf],
                 dtype=np.float32),
    ]
    # exact halfway points between fp16 neighbours (ties to even)
    base = np.arange(0, 65504, 0.5, dtype=np.float16)[:-1].astype(np.float32)
    with np.errstate(over="ignore"):
        nxt = np.nextafter(base.astype(np.float16), np.float16(np.inf)).astype(np.float32)
    parts.append(((base + nxt) * 0.5).astype(np.float32))
    x = np.concatenate(parts)
    ours = oracle.f32_to_f16(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (reference tree absent)")
def test_codec_matches_compiled_reference():
    ref = oracle.ref()
    ref.kvref_float_to_kv.restype = ctypes.c_uint16
    ref.kvref_float_to_kv.argtypes = [ctypes.c_float]
    ref.kvref_kv_to_float.restype = ctypes.c_float
    ref.kvref_kv_to_float.argtypes = [ctypes.c_uint16]
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10,
                        np.array([np.nan, -np.nan, np.inf, 1e-8, -1e-7], dtype=np.float32)])
    ours = oracle.f32_to_f16(x)
    for v, o in zip(x, ours):
        assert ref.kvref_float_to_kv(float(v)) == o
    for c in range(0, 65536, 7):
        a = ref.kvref_kv_to_float(c)
        b = oracle.lib().kvo_f16_to_f32(c)
        assert (math.isnan(a) and math.isnan(b)) or a == b


# ---- synthetic generator ------------------------------------------------------

def test_synth_generator_properties():
    vals = helpers.to_f32(oracle.synth_rows(200000, 1234, 0, 256))
    assert np.all(np.abs(vals) <= 4.0)
    assert abs(float(vals.mean())) < 0.02
    assert abs(float(vals.std()) - 2.0 / math.sqrt(3.0)) < 0.02     # Irwin-Hall(4) scaled by 2^-15
    # Distinct seeds and rows give distinct streams.
    a = oracle.synth_rows(1000, 1, 0, 64)
    b = oracle.synth_rows(1000, 2, 0, 64)
    assert np.mean(a == b) < 0.05


def test_synth_generator_closed_form():
    # v = sum of the four 16-bit fields of h minus 131070, h = mix(mix(seed + row*phi) + col)
    mask = (1 << 64) - 1

    def mix(z):
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask
        return z ^ (z >> 31)

    for seed, row, col in [(0, 0, 0), (99, 12345, 7), (2 ** 63 + 5, 2 ** 40 + 3, 255)]:
        h = mix((mix((seed + row * 0x9E3779B97F4A7C15) & mask) + col) & mask)
        v = sum((h >> s) & 0xFFFF for s in (0, 16, 32, 48)) - 131070
        expected = np.float32(v / 32768.0).astype(np.float16).view(np.uint16)
        assert oracle.lib().kvo_synth(seed, row, col) == expected


# ---- attention ----------------------------------------------------------------

def test_reference_attention_closed_form():
    # tests/reference/kv_reference_test.cpp:45-95
    L, H, D, T = 1, 1, 2, 2
    kv = np.zeros(L * 2 * T * H * D, dtype=np.uint16)
    f = lambda v: np.float16(v).view(np.uint16)
    # K token0 = (0,0), token1 = (1,0); V token0 = (1,2), token1 = (3,4)
    kv[2] = f(1.0)                 # K t1 d0  (offset ((0*2+0)*2+1)*1*2+0)
    kv[4], kv[5] = f(1.0), f(2.0)  # V t0
    kv[6], kv[7] = f(3.0), f(4.0)  # V t1
    out = oracle.reference_attention(L, H, D, kv, T, np.array([1.0, 0.0], dtype=np.float32))
    w = math.exp(1.0 / math.sqrt(2.0))
    assert abs(out[0] - (1 + 3 * w) / (1 + w)) < 1e-6
    assert abs(out[1] - (2 + 4 * w) / (1 + w)) < 1e-6
    with pytest.raises(ValueError):
        oracle.reference_attention(L, H, D, kv, 0, np.array([1.0, 0.0], dtype=np.float32))


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (reference tree absent)")
def test_reference_attention_matches_compiled_reference():
    ref = oracle.ref()
    ref.kvref_reference_attention.restype = ctypes.c_int
    ref.kvref_reference_attention.argtypes = [ctypes.c_uint32] * 3 + [ctypes.c_void_p, ctypes.c_uint32,
                                                                        ctypes.c_void_p, ctypes.c_void_p]
    rng = np.random.default_rng(3)
    for (L, H, D, T) in [(2, 2, 8, 37), (1, 4, 64, 300)]:
        kv = rng.standard_normal(L * 2 * T * H * D).astype(np.float16).view(np.uint16)
        q = rng.standard_normal(L * H * D).astype(np.float32)
        ours = oracle.reference_attention(L, H, D, kv, T, q)
        theirs = np.zeros_like(ours)
        assert ref.kvref_reference_attention(L, H, D, kv.ctypes.data, T, q.ctypes.data, theirs.ctypes.data)
        assert np.max(np.abs(ours - theirs)) <= 1e-6


def _brute_force_gqa(kv_f64, q_f64, scale, group):
    """float64 textbook attention: kv [2][T][H][D], q [QH][D]."""
    K, V = kv_f64[0], kv_f64[1]
    out = np.zeros_like(q_f64)
    for j in range(q_f64.shape[0]):
        h = j // group
        s = K[:, h, :] @ q_f64[j] * scale
        p = np.exp(s - s.max())
        out[j] = (p[:, None] * V[:, h, :]).sum(0) / p.sum()
    return out


@pytest.mark.parametrize("T,H,G,D", [(1, 1, 1, 4), (17, 2, 4, 8), (100, 4, 8, 64), (513, 4, 8, 64)])
def test_paged_decode_oracle_brute_force(T, H, G, D):
    rng = np.random.default_rng(T)
    L, layer = 2, 1
    alloc = helpers.SlotAllocator(256, 32, seed=T)
    table = helpers.hetero_table(T, alloc)
    pools = oracle.HostPools(L, H, D, 256, 32)
    kv = rng.standard_normal((L, 2, T, H, D)).astype(np.float16).view(np.uint16)
    for e in table:
        pools.append_tokens(kv, T, e["logical_token_begin"], e["kind"], e["slot"], 0, e["valid_tokens"])
    q = rng.standard_normal(H * G * D).astype(np.float16).view(np.uint16)
    scale = 1.0 / math.sqrt(D)
    got = pools.paged_decode(table, T, layer, H * G, q, scale, f32=True)
    want = _brute_force_gqa(helpers.to_f32(kv[layer]).astype(np.float64),
                            helpers.to_f32(q).astype(np.float64).reshape(H * G, D), scale, G)
    assert np.max(np.abs(got - want.reshape(-1))) < 2e-5


def test_paged_decode_oracle_equals_reference_attention_per_head():
    """GQA decode of q head j == the reference's MHA attention on kv head j/G
    (kv_reference.cpp:136-234 with the test ReferenceModel head map,
    tests/cuda/cuda_model_runner_test.cpp:339-374)."""
    rng = np.random.default_rng(5)
    L, H, G, D, T = 1, 2, 3, 16, 90
    alloc = helpers.SlotAllocator(64, 8)
    table = helpers.hetero_table(T, alloc)
    pools = oracle.HostPools(L, H, D, 64, 8)
    kv = rng.standard_normal((L, 2, T, H, D)).astype(np.float16).view(np.uint16)
    for e in table:
        pools.append_tokens(kv, T, e["logical_token_begin"], e["kind"], e["slot"], 0, e["valid_tokens"])
    q = rng.standard_normal(H * G * D).astype(np.float16).view(np.uint16)
    got = pools.paged_decode(table, T, 0, H * G, q, 1.0 / math.sqrt(D), f32=True).reshape(H * G, D)
    for j in range(H * G):
        query = np.zeros((L, H, D), dtype=np.float32)
        query[0, j // G] = helpers.to_f32(q.reshape(H * G, D)[j])
        ref = oracle.reference_attention(L, H, D, kv.reshape(-1), T, query.reshape(-1)).reshape(L, H, D)
        assert np.max(np.abs(ref[0, j // G] - got[j])) < 1e-5


def test_gqa_closed_form_engine_test():
    """tests/cuda/cuda_engine_kv_backend_test.cpp:96-129 (2 q heads, 1 kv head,
    D=2, two layers), tolerance 0.035 as in :242-248."""
    pools = oracle.HostPools(2, 1, 2, 16, 2)
    history = []
    f16 = lambda v: np.float16(v).view(np.uint16)
    queries = np.array([f16(0.5), f16(0.25), f16(-0.2), f16(0.4)], dtype=np.uint16)
    scale = 1.0 / math.sqrt(2.0)
    slots = iter(range(16))
    pages = []
    for token in range(12):
        pos = len(history)
        if pos % 8 == 0:
            pages.append(next(slots))
        for layer in range(2):
            lo = 0.02 if layer == 1 else 0.0
            key = np.array([f16(0.1 * (token + 1) + lo), f16(-0.05 * token + lo * 0.5)], dtype=np.uint16)
            val = np.array([f16(token + 1 + lo * 10.0), f16((token + 1) * 0.5 - lo * 5.0)], dtype=np.uint16)
            pools.write_layer_token(0, pages[-1], pos % 8, layer, key, val)
        history.append(token)
        n = len(history)
        table = np.array([(pages[i], 1, 8 * i, min(8, n - 8 * i), 8, 0) for i in range(len(pages))],
                         dtype=helpers.DESC)
        got = helpers.to_f32(pools.paged_decode(table, n, 1, 2, queries, scale))
        # referenceOutput (cuda_engine_kv_backend_test.cpp:96-129) is the last layer (1)
        qs = [[0.5, 0.25], [-0.2, 0.4]]
        exp = []
        for qh in range(2):
            scores = [(qs[qh][0] * (0.1 * (t + 1) + 0.02) + qs[qh][1] * (-0.05 * t + 0.01)) * scale
                      for t in history]
            m = max(scores)
            w = [math.exp(s - m) for s in scores]
            den = sum(w)
            exp += [sum(wi * (t + 1 + 0.2) for wi, t in zip(w, history)) / den,
                    sum(wi * ((t + 1) * 0.5 - 0.1) for wi, t in zip(w, history)) / den]
        assert np.max(np.abs(got - np.array(exp))) < 0.035


# ---- page copies ------------------------------------------------------------------

def test_gather_append_promotion_closed_form():
    """Byte-exact gather of makeKv data before and after promotion and after a
    partial-tail COW copy (tests/cuda/cuda_kv_test.cpp:287-391)."""
    L, H, D = 2, 2, 8
    pools = oracle.HostPools(L, H, D, 16, 2)
    T = 70
    data = helpers.make_kv_closed_form(L, H, D, 0, T)
    entries = []
    for i in range(9):
        n = min(8, T - 8 * i)
        pools.append_tokens(data, T, 8 * i, 0, i, 0, n)
        entries.append((i, 1, 8 * i, n, 8, 0))
    table = np.array(entries, dtype=helpers.DESC)
    assert np.array_equal(pools.gather(table, T), data.reshape(-1))
    pools.promote(list(range(8)), 1)
    promoted = np.array([(1, 1, 0, 64, 64, 1), (8, 1, 64, 6, 8, 0)], dtype=helpers.DESC)
    assert np.array_equal(pools.gather(promoted, T), data.reshape(-1))
    # COW: copy the 6-token tail into a fresh micro page and gather through it.
    pools.copy_page_tokens(0, 8, 0, 12, 6)
    cow = promoted.copy()
    cow[1]["slot"] = 12
    assert np.array_equal(pools.gather(cow, T), data.reshape(-1))
