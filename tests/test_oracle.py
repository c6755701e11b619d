"""Pins the CPU oracle before anything is checked against it.

Sources of truth, in order: the reference's own known-answer tests
(AI/codes/local-llm/test/LaunchAddTest.cpp), the storage formats through the independent encoders
in qgen.py, numpy's IEEE binary16 conversion, and mathematical identities (exact sums, linearity,
brute-force top-k).  No test here retypes the oracle's own formula.
"""
import numpy as np
import pytest

import qgen
from qgen import Q4_0, Q5_0, Q8_0, Q4_K, Q6_K, f16_bits

TYPES = [Q4_0, Q5_0, Q8_0, Q4_K, Q6_K]


# ---- binary16 ---------------------------------------------------------------------------------

def test_f16_decode_exhaustive(orc):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f16_encode_matches_ieee_rne(orc):
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, size=400_000, dtype=np.uint64).astype(np.uint32)
    # concentrate on the binary16 range, subnormals, the overflow edge and exact halfway points
    exps = rng.integers(100, 145, size=200_000).astype(np.uint32)
    near = (exps << 23) | rng.integers(0, 2**23, size=200_000).astype(np.uint32)
    halfway = (np.arange(1, 2**10, dtype=np.uint32) << 13) | 0x1000 | (np.uint32(120) << 23)
    edges = np.array([0x477ff000, 0x477fefff, 0x477fe000, 0x38800000, 0x387fffff, 0x33000000,
                      0x33000001, 0x32ffffff, 0x7f800000, 0xff800000, 0x80000000, 0], np.uint32)
    allbits = np.concatenate([bits, near, halfway, near | 0x80000000, edges])
    f = allbits.view(np.float32)
    got = orc.f32_to_f16(f)
    with np.errstate(over="ignore"):  # values past the f16 range become infinities, as they should
        ref = f.astype(np.float16).view(np.uint16)
    isnan = np.isnan(f)
    assert np.array_equal(got[~isnan], ref[~isnan])
    assert np.all((got[isnan] & 0x7c00) == 0x7c00) and np.all(got[isnan] & 0x3ff)


# ---- block codecs against the independent encoders -------------------------------------------

@pytest.mark.parametrize("qtype", TYPES)
def test_dequant_matches_format(orc, qtype):
    rng = np.random.default_rng(100 + qtype)
    nb = 4096 if qtype in (Q4_0, Q5_0, Q8_0) else 512
    packed, vals = qgen.random_blocks(qtype, nb, rng)
    n = vals.size
    got = orc.dequant_f32(qtype, packed, n)
    assert np.array_equal(got.view(np.uint32), vals.astype(np.float32).view(np.uint32))
    got16 = orc.dequant_f16(qtype, packed, n)
    assert np.array_equal(got16, vals.astype(np.float16).view(np.uint16))


def test_q4k_every_scale_and_min_field(orc):
    """All 64 values of every 6-bit scale and min, at every sub-block (both packing branches)."""
    for j in range(8):
        for v in range(64):
            sc = np.full((1, 8), (v * 7 + 3) % 64)
            mn = np.full((1, 8), (v * 5 + 1) % 64)
            sc[0, j] = v
            mn[0, j] = 63 - v
            q = np.zeros((1, 256))
            packed = qgen.pack_q4_k(f16_bits([1.0]), f16_bits([1.0]), sc, mn, q)
            assert orc.q4k_scale_min(j, packed[4:16].tobytes()) == (v, 63 - v)
            # value of sub-block j with q = 0 is -dmin*m
            vals = orc.dequant_f32(Q4_K, packed, 256)
            assert np.all(vals[32 * j:32 * j + 32] == -float(63 - v))


def test_q6k_every_bit_position(orc):
    """Each element's 6-bit value can reach every value 0..63 independently."""
    rng = np.random.default_rng(7)
    for trial in range(64):
        q = (np.arange(256) * 37 + trial * 11) % 64 - 32
        q = q.reshape(1, 256)
        sc = rng.integers(-128, 128, size=(1, 16))
        d = f16_bits([0.5])
        packed = qgen.pack_q6_k(d, sc, q)
        vals = orc.dequant_f32(Q6_K, packed, 256)
        assert np.array_equal(vals, qgen.value_q6_k(d, sc, q).reshape(-1))


def test_q5_0_every_high_bit(orc):
    for e in range(32):
        q = np.full((1, 32), 5)
        q[0, e] = 16 + 5
        d = f16_bits([1.0])
        vals = orc.dequant_f32(Q5_0, qgen.pack_q5_0(d, q), 32)
        exp = np.full(32, -11.0, np.float32)
        exp[e] = 5.0
        assert np.array_equal(vals, exp)


# ---- the reference's known-answer tests (LaunchAddTest.cpp) -----------------------------------

def _u16(b, off, v):
    b[off] = v & 0xFF
    b[off + 1] = v >> 8


def q4k_kat_block():
    """LaunchAddTest.cpp:711-756: d=1, dmin=0.5, sub-block 0 scale 3 / min 2, q=5 -> w=14."""
    w = np.zeros(144, np.uint8)
    _u16(w, 0, 0x3C00)
    _u16(w, 2, 0x3800)
    w[4 + 0] = 3
    w[4 + 4] = 2
    w[16:48] = 0x05
    return w


def q6k_kat_block():
    """LaunchAddTest.cpp:758-803: stored q = 35, scale 2, d = 1 -> w = 6 for the first 32."""
    w = np.zeros(210, np.uint8)
    w[0:32] = 0x03
    w[128:160] = 0x02
    w[192] = 2
    w[193] = 2
    _u16(w, 208, 0x3C00)
    return w


def kat_x():
    x = np.zeros(256, np.float32)
    x[0] = 127.0
    x[1:32] = 1.0
    return x


@pytest.mark.parametrize("qtype,block,expected", [(Q4_K, q4k_kat_block, 14.0 * 158.0),
                                                  (Q6_K, q6k_kat_block, 6.0 * 158.0)])
def test_kat_q8_1_matmul(orc, qtype, block, expected):
    w = block()
    x = kat_x()
    xq = orc.quantize_q8_1(x, 256)
    y = orc.matmul_q8_1(qtype, w, w.size, xq, 1, 256, 1)
    assert abs(y[0, 0] - expected) <= 1e-3
    # the f32-activation path sees the same dequantized weights
    y32 = orc.matmul_f64(qtype, w, w.size, x, 1, 256)
    assert abs(y32[0, 0] - expected) <= 1e-3


def test_kat_q8_0_matmul_rows(orc):
    """LaunchAddTest.cpp:186-240: row 0 all ones, row 1 alternating (2, -1); m = 3."""
    w = np.zeros(68, np.uint8)
    for row in range(2):
        _u16(w, row * 34, 0x3C00)
        for k in range(32):
            q = 1 if row == 0 else (2 if k % 2 == 0 else -1)
            w[row * 34 + 2 + k] = q & 0xFF
    x = np.array(list(range(1, 33)) + [-v for v in range(1, 33)] + [1, -1] * 16, np.float32).reshape(3, 32)
    y = orc.matmul_f64(Q8_0, w, 34, x, 2, 32)
    for r in range(3):
        e0 = float(x[r].sum())
        e1 = float(sum(x[r, k] * (2 if k % 2 == 0 else -1) for k in range(32)))
        assert abs(y[r, 0] - e0) <= 1e-5 and abs(y[r, 1] - e1) <= 1e-5


def test_kat_q8_0_via_q8_1(orc):
    """LaunchAddTest.cpp:242-299: x[0] = +-127, x[k] = +-k, so Q8_1 is exact with d = 1."""
    w = np.zeros(68, np.uint8)
    for row in range(2):
        _u16(w, row * 34, 0x3C00)
        for k in range(32):
            q = 1 if row == 0 else (2 if k % 2 == 0 else -1)
            w[row * 34 + 2 + k] = q & 0xFF
    x = np.zeros((2, 32), np.float32)
    x[0, 0], x[1, 0] = 127, -127
    x[0, 1:] = np.arange(1, 32)
    x[1, 1:] = -np.arange(1, 32)
    xq = orc.quantize_q8_1(x, 32)
    y = orc.matmul_q8_1(Q8_0, w, 34, xq, 2, 32, 2)
    for r in range(2):
        e0 = float(x[r].sum())
        e1 = float(sum(x[r, k] * (2 if k % 2 == 0 else -1) for k in range(32)))
        assert abs(y[r, 0] - e0) <= 1e-5 and abs(y[r, 1] - e1) <= 1e-5


def test_kat_q8_1_block_sums(orc):
    """LaunchAddTest.cpp:679-709: x = 0.01 except x[0] = 1 -> d*sum(q) = 158/127, raw 1.31."""
    x = np.full(32, 0.01, np.float32)
    x[0] = 1.0
    s_q = qgen.f16_val(orc.quantize_q8_1(x, 32, False)[2:4].view("<u2"))[0]
    s_raw = qgen.f16_val(orc.quantize_q8_1(x, 32, True)[2:4].view("<u2"))[0]
    assert abs(s_q - 158.0 / 127.0) <= 1e-3
    assert abs(s_raw - 1.31) <= 1e-3


# ---- Q8_1 quantizer invariants -----------------------------------------------------------------

def test_q8_1_invariants(orc):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((7, 96)).astype(np.float32)
    x[2, 32:64] = 0.0  # an all-zero block
    xq = orc.quantize_q8_1(x, 96).reshape(7, 3, 36)
    for r in range(7):
        for b in range(3):
            blk = xq[r, b]
            d = qgen.f16_val(blk[0:2].view("<u2"))[0]
            q = blk[4:].view(np.int8).astype(np.int64)
            xs = x[r, 32 * b:32 * b + 32]
            amax = np.abs(xs).max()
            if amax == 0:
                assert d == 0 and np.all(q == 0)
                continue
            assert d == np.float16(np.float32(amax) / np.float32(127))
            assert np.abs(q).max() == 127 and np.all(np.abs(q) <= 127)
            assert q[np.argmax(np.abs(xs))] == np.sign(xs[np.argmax(np.abs(xs))]) * 127
            # q is the nearest integer to x/d_exact (within rounding of the f32 reciprocal)
            assert np.max(np.abs(q - xs * 127.0 / amax)) <= 0.5 + 1e-4
            s = qgen.f16_val(blk[2:4].view("<u2"))[0]
            assert s == np.float16(np.float32(np.float32(amax) / np.float32(127)) * np.float32(q.sum()))


def test_q8_1_partial_block_zero_padded(orc):
    x = np.arange(1, 41, dtype=np.float32).reshape(1, 40)
    xq = orc.quantize_q8_1(x, 40)
    assert xq.size == 72
    q2 = xq[36 + 4:].view(np.int8)
    assert np.all(q2[8:] == 0) and q2[7] == 127


def test_q4k_q8_1_min_term_identity(orc):
    """When the stored block sum is exact (d = 1, integer x), the Q8_1 block-dot with its
    min compensation equals the plain dot with the dequantized weights."""
    w, rb, vals = qgen.random_matrix(Q4_K, 8, 512, seed=5)
    rng = np.random.default_rng(9)
    x = rng.integers(-40, 41, size=(3, 512)).astype(np.float32)
    x[:, ::32] = 127.0  # amax = 127 in every block -> d = 1 exactly, q = x
    xq = orc.quantize_q8_1(x, 512)
    y = orc.matmul_q8_1(Q4_K, w, rb, xq, 8, 512, 3)
    ref = x.astype(np.float64) @ vals.astype(np.float64).T
    assert np.max(np.abs(y - ref)) <= 1e-9 * np.max(np.abs(ref)) + 1e-9


# ---- contractions ------------------------------------------------------------------------------

@pytest.mark.parametrize("qtype", TYPES)
def test_matmul_truth_matches_closed_form(orc, qtype):
    in_dim = 512
    w, rb, vals = qgen.random_matrix(qtype, 48, in_dim, seed=20 + qtype)
    x = qgen.random_x(3, in_dim, seed=30)
    y = orc.matmul_f64(qtype, w, rb, x, 48, in_dim)
    ref = x.astype(np.float64) @ vals.astype(np.float64).T
    assert np.max(np.abs(y - ref)) <= 1e-12 * np.max(np.abs(ref))


@pytest.mark.parametrize("qtype", TYPES)
def test_fp32_orders_within_tolerance(orc, qtype):
    in_dim = 2048
    w, rb, _ = qgen.random_matrix(qtype, 64, in_dim, seed=40 + qtype)
    x = qgen.random_x(2, in_dim, seed=41)
    truth = orc.matmul_f64(qtype, w, rb, x, 64, in_dim)
    assert qgen.normwise_rel_err(orc.matmul_f32(qtype, w, rb, x, 64, in_dim, 2), truth) < 1e-5
    assert qgen.normwise_rel_err(orc.matmul_lane32(qtype, w, rb, x, 64, in_dim), truth) < 1e-5


def test_matmul_linearity(orc):
    w, rb, _ = qgen.random_matrix(Q4_K, 16, 768, seed=50)
    x = qgen.random_x(2, 768, seed=51)
    y = orc.matmul_f64(Q4_K, w, rb, x, 16, 768)
    y2 = orc.matmul_f64(Q4_K, w, rb, (x[0] * 2.0 - x[1] * 0.5).reshape(1, -1), 16, 768)
    assert np.max(np.abs(y2[0] - (2.0 * y[0] - 0.5 * y[1]))) <= 1e-5 * np.max(np.abs(y2))


def test_unsupported_type_rejected(orc):
    with pytest.raises(ValueError):
        orc.matmul_f64(3, np.zeros(64, np.uint8), 32, np.zeros(32, np.float32), 1, 32)
    with pytest.raises(ValueError):
        orc.matmul_f64(Q4_K, np.zeros(144, np.uint8), 144, np.zeros(128, np.float32), 1, 128)


def test_gemv_add_accumulates(orc):
    w, rb, vals = qgen.random_matrix(Q8_0, 10, 64, seed=60)
    x = qgen.random_x(1, 64, seed=61)[0]
    y0 = np.linspace(-1, 1, 10).astype(np.float32)
    y = orc.gemv_add(Q8_0, w, rb, x, y0, 10, 64)
    assert np.allclose(y, y0 + vals.astype(np.float64) @ x, rtol=0, atol=1e-5)


# ---- MoE ---------------------------------------------------------------------------------------

def test_router_bruteforce(orc):
    rng = np.random.default_rng(70)
    logits = rng.standard_normal((16, 64)).astype(np.float32)
    idx, w = orc.router_topk(logits, 6, 1.0)
    for t in range(16):
        order = sorted(range(64), key=lambda e: (-logits[t, e], e))[:6]
        assert list(idx[t]) == order
        p = np.exp(logits[t].astype(np.float64) - logits[t].max())
        p /= p.sum()
        assert np.allclose(w[t], p[order], rtol=1e-5, atol=1e-7)
    idx2, w2 = orc.router_topk(logits, 6, 2.5)
    assert np.array_equal(idx2, idx) and np.allclose(w2, 2.5 * w, rtol=1e-6)


def test_router_ties_and_nonfinite(orc):
    logits = np.zeros((1, 8), np.float32)
    logits[0, [5, 2, 7]] = 3.0  # three-way tie: lowest index first
    logits[0, 1] = np.nan
    logits[0, 4] = np.inf      # non-finite -> -inf, never picked while finite ones remain
    idx, w = orc.router_topk(logits, 4, 1.0)
    assert list(idx[0]) == [2, 5, 7, 0]
    assert np.all(w[0, :3] == w[0, 0]) and w[0, 3] < w[0, 0]
    allnan = np.full((1, 4), np.nan, np.float32)
    idx, w = orc.router_topk(allnan, 2, 1.0)
    assert list(idx[0]) == [0, 1] and np.all(w == 0)


def _silu_mul(g, u):
    with np.errstate(over="ignore"):  # exp(-g) overflows to inf for very negative g: silu is then 0
        return g / (1.0 + np.exp(-g)) * u


def test_swiglu_paths(orc):
    E, ffn, hid = 3, 40, 256
    wg, rb, vg = qgen.random_matrix(Q4_K, E * ffn, hid, seed=80)
    wu, _, vu = qgen.random_matrix(Q4_K, E * ffn, hid, seed=81)
    x = qgen.random_x(1, hid, seed=82)[0] * 10
    eb = ffn * rb
    ids = np.array([2, -1, 0], np.int32)
    act = orc.swiglu_indexed(Q4_K, wg, wu, eb, eb, rb, rb, x, ids, ffn, hid)
    for r, e in enumerate(ids):
        if e < 0:
            assert np.all(act[r] == 0)
            continue
        g = vg[e * ffn:(e + 1) * ffn].astype(np.float64) @ x
        u = vu[e * ffn:(e + 1) * ffn].astype(np.float64) @ x
        assert np.allclose(act[r], _silu_mul(g, u), rtol=1e-6, atol=1e-9)
    # the shared-expert (non-indexed) form on expert 2's slice
    a2 = orc.swiglu(Q4_K, wg[2 * eb:3 * eb], wu[2 * eb:3 * eb], rb, rb, x, ffn, hid)
    assert np.array_equal(a2, act[0])


def test_down_ordered(orc):
    E, hid, ffn = 4, 24, 64
    wd, rb, vd = qgen.random_matrix(Q5_0, E * hid, ffn, seed=90)
    act = qgen.random_x(3, ffn, seed=91)
    ids = np.array([3, -1, 1], np.int32)
    rw = np.array([0.5, 9.0, -0.25], np.float32)
    out0 = np.linspace(-1, 1, hid).astype(np.float32)
    out = orc.down_indexed_ordered(Q5_0, wd, hid * rb, rb, act, ids, rw, out0, hid, ffn)
    ref = out0.astype(np.float64).copy()
    for r, e in enumerate(ids):
        if e >= 0:
            ref += rw[r] * (vd[e * hid:(e + 1) * hid].astype(np.float64) @ act[r])
    assert np.allclose(out, ref, rtol=1e-6, atol=1e-6)


def test_argmax_lowest_index_on_ties(orc):
    v = np.array([1, 5, np.nan, 5, -np.inf, 2], np.float32)
    assert orc.argmax(v) == 1
    assert orc.argmax(np.full(5, -np.inf, np.float32)) == 0


def test_first_use_from_threads():
    """The first calls into the oracle's library may come from a thread pool (the CPU baseline legs
    do this); each must see the declared signatures: a call through a function whose argument types
    are not yet set passes its pointers as 32-bit ints and crashes.  Fresh interpreters (the library
    not yet loaded; a crash shows as a status, not as the test runner's end), 16 threads released
    together, and a tiny thread switch interval so a switch lands inside the loader."""
    import os
    import subprocess
    import sys
    here = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(here)
    code = (
        "import sys; sys.path[:0] = [%r, %r]\n"
        "sys.setswitchinterval(1e-6)\n"
        "import threading, numpy as np, oracle\n"
        "from concurrent.futures import ThreadPoolExecutor\n"
        "h = np.arange(4096, dtype=np.uint16)\n"
        "ref = h.view(np.float16).astype(np.float32)\n"
        "gate = threading.Barrier(16)\n"
        "def one(_):\n"
        "    gate.wait()\n"
        "    got = oracle.f16_to_f32(h)\n"
        "    return bool(np.array_equal(got[:1024], ref[:1024]))\n"
        "with ThreadPoolExecutor(16) as ex:\n"
        "    ok = list(ex.map(one, range(16)))\n"
        "assert all(ok)\n"
    ) % (os.path.join(root, "oracle"), root)
    for _ in range(6):
        r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, (r.returncode, r.stderr[-2000:])
