"""The Q8_1-activation variants (kernel.cu:1395-1765, 1873-2242, 2405-2660; launch.cu:209-455, 546-560).

The reference has no tests of these kernels; they reuse the Q8_1 quantizer and block-dot semantics
that its KATs pin (tests/golden, test_oracle.py).  The oracle is pinned here on the CPU: the MMQ
layout is a permutation of the quantizer's blocks, the MMQ matmul equals the row-layout matmul, and
the routed SwiGLU / down forms equal float64 products of the dequantized operands (with the Q4_K
stored-sum term).  The GPU tests compare the HIP entry points with the oracle at C5's shapes.
"""
import numpy as np
import pytest

import oracle as orc
import qgen
from blog_amd import qlin
from qgen import Q4_K, Q5_0, Q6_K, Q8_0, normwise_rel_err
from test_embed_mla import q4k_min_coeffs


def decode_rows(xq, in_dim):
    """(values [m, in_dim], S - in-order block sums [m, nb]) of standard Q8_1 rows."""
    bpr = in_dim // 32
    blk = np.asarray(xq, np.uint8).reshape(-1, bpr, 36)
    d = blk[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float32)
    s = blk[:, :, 2:4].copy().view(np.float16)[..., 0].astype(np.float32)
    vals = d[:, :, None] * blk[:, :, 4:].view(np.int8).astype(np.float32)
    dsum = np.add.accumulate(vals, axis=2, dtype=np.float32)[:, :, -1]
    return vals.reshape(-1, in_dim), s - dsum


def ref_dot(qtype, w, rb, vals, n, xq, in_dim):
    """float64 W . x_q8_1 rows of the dequantized operands, with Q4_K's stored-sum min term."""
    xv, corr = decode_rows(xq, in_dim)
    y = xv.astype(np.float64) @ vals.astype(np.float64).T
    if qtype == Q4_K:
        y += corr.astype(np.float64) @ q4k_min_coeffs(w, n, in_dim).astype(np.float64).T
    return y


# ---- the oracle ----------------------------------------------------------------------------------

@pytest.mark.parametrize("in_dim,m,raw", [(4096, 5, False), (300, 3, False), (512, 2, True)])
def test_oracle_mmq_layout_is_the_blocks_regrouped(in_dim, m, raw):
    x = qgen.random_x(m, in_dim, seed=in_dim)
    groups = (in_dim + 127) // 128
    got = orc.quantize_q8_1_mmq(x, in_dim, raw).reshape(groups, m, 144)
    pad = np.zeros((m, groups * 128), np.float32)
    pad[:, :in_dim] = x
    blocks = orc.quantize_q8_1(pad, groups * 128, raw).reshape(m, groups, 4, 36)
    for g in range(groups):
        for r in range(m):
            assert np.array_equal(got[g, r, :16].reshape(4, 4), blocks[r, g, :, :4])
            assert np.array_equal(got[g, r, 16:].reshape(4, 32), blocks[r, g, :, 4:])


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
def test_oracle_mmq_matmul_equals_row_layout(qtype):
    w, rb, _ = qgen.random_matrix(qtype, 40, 768, seed=5 + qtype)
    x = qgen.random_x(6, 768, seed=6)
    y = orc.matmul_q8_1_mmq(qtype, w, rb, orc.quantize_q8_1_mmq(x, 768), 40, 768, 6)
    assert np.array_equal(y, orc.matmul_q8_1(qtype, w, rb, orc.quantize_q8_1(x, 768), 40, 768, 6))


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
def test_oracle_swiglu_q8_1_against_dequantized(qtype):
    E, ffn, hid = 3, 48, 512
    wg, rb, vg = qgen.random_matrix(qtype, E * ffn, hid, seed=10 + qtype)
    wu, _, vu = qgen.random_matrix(qtype, E * ffn, hid, seed=11 + qtype)
    eb = ffn * rb
    xq = orc.quantize_q8_1(qgen.random_x(1, hid, seed=12), hid)
    ids = np.array([2, -1, 0], np.int32)
    act = orc.swiglu_indexed_q8_1(qtype, wg, wu, eb, eb, rb, rb, xq, ids, ffn, hid)
    assert not act[1].any()
    for r, e in enumerate(ids):
        if e < 0:
            continue
        sl = slice(e * ffn, (e + 1) * ffn)
        g = ref_dot(qtype, wg[e * eb:(e + 1) * eb], rb, vg[sl], ffn, xq, hid)[0]
        u = ref_dot(qtype, wu[e * eb:(e + 1) * eb], rb, vu[sl], ffn, xq, hid)[0]
        assert normwise_rel_err(act[r], g / (1 + np.exp(-g)) * u) <= 1e-6


@pytest.mark.parametrize("qtype,ffn", [(Q5_0, 160), (Q8_0, 160), (Q4_K, 256), (Q6_K, 256)])
def test_oracle_down_q8_1_against_dequantized(qtype, ffn):
    E, hid, k = 4, 24, 3
    wd, rb, vd = qgen.random_matrix(qtype, E * hid, ffn, seed=20 + qtype)
    eb = hid * rb
    act = qgen.random_x(k, ffn, seed=21)
    aq = orc.quantize_q8_1(act, ffn)
    ids = np.array([1, -1, 3], np.int32)
    rw = np.array([0.5, 9.0, 0.25], np.float32)
    out0 = np.linspace(-1, 1, hid)
    got = orc.down_q8_1_indexed_accum(qtype, wd, eb, rb, aq, ids, rw, out0, hid, ffn)
    ref = out0.copy()
    for r, e in enumerate(ids):
        if e >= 0:
            ref += rw[r] * ref_dot(qtype, wd[e * eb:(e + 1) * eb], rb, vd[e * hid:(e + 1) * hid], hid,
                                   aq[r * (ffn // 32) * 36:(r + 1) * (ffn // 32) * 36], ffn)[0]
    assert normwise_rel_err(got - out0, ref - out0) <= 1e-6
    # the f32 form quantizes each route's act first
    assert np.array_equal(orc.down_q8_1_indexed_accum(qtype, wd, eb, rb, act, ids, rw, out0, hid, ffn, f32_act=True),
                          got)


# ---- the HIP entry points ------------------------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("in_dim,m,raw", [(4096, 5, False), (300, 3, False), (512, 2, True)])
def test_quantize_mmq_bit_exact(in_dim, m, raw):
    from gpu_util import banner, bind_stream, dev, host
    import torch
    x = qgen.random_x(m, in_dim, seed=30 + in_dim)
    x[0, :32] = 0.0
    banner(f"quantize mmq in_dim={in_dim} m={m}")
    bind_stream()
    n = (in_dim + 127) // 128 * m * 144
    xq = torch.empty(n, dtype=torch.uint8, device="cuda")
    qlin.call("qlin_launch_quantize_q8_1_mmq", dev(x), xq, in_dim, m, int(raw))
    assert np.array_equal(host(xq), orc.quantize_q8_1_mmq(x, in_dim, raw))


@pytest.mark.gpu
@pytest.mark.parametrize("qtype,m", [(Q4_K, 7), (Q6_K, 3)])
def test_matmul_mmq_and_gemv_q8_1(qtype, m):
    from gpu_util import banner, bind_stream, dev, empty_f32, host
    w, rb, _ = qgen.random_matrix(qtype, 96, 1024, seed=40 + qtype)
    x = qgen.random_x(m, 1024, seed=41)
    banner(f"matmul mmq type={qtype} m={m}")
    bind_stream()
    xm = orc.quantize_q8_1_mmq(x, 1024)
    y = empty_f32(m, 96)
    qlin.call("qlin_launch_quant_matmul_q8_1_mmq", qtype, dev(w), rb, dev(xm), y, 96, 1024, m)
    assert normwise_rel_err(host(y), orc.matmul_q8_1_mmq(qtype, w, rb, xm, 96, 1024, m)) <= 1e-5
    xr = orc.quantize_q8_1(x[:1], 1024)
    y1 = empty_f32(96)
    qlin.call("qlin_launch_quant_gemv_q8_1", qtype, dev(w), rb, dev(xr), y1, 96, 1024)
    assert normwise_rel_err(host(y1), orc.matmul_q8_1(qtype, w, rb, xr, 96, 1024, 1)[0]) <= 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
def test_swiglu_indexed_block_and_q8_1(qtype):
    """C5's routed gate/up ([1408, 2048] per expert, 6 routes, one empty) through the block form
    (f32 x) and the Q8_1-x form."""
    from gpu_util import banner, bind_stream, dev, empty_f32, host
    E, ffn, hid, k = 8, 1408, 2048, 6
    wg, rb, _ = qgen.random_matrix(qtype, E * ffn, hid, seed=50 + qtype)
    wu, _, _ = qgen.random_matrix(qtype, E * ffn, hid, seed=51 + qtype)
    eb = ffn * rb
    x = qgen.random_x(1, hid, seed=52)[0]
    ids = np.array([3, 0, -1, 7, 3, 5], np.int32)
    banner(f"swiglu block / q8_1 type={qtype}")
    bind_stream()
    dg, du, di = dev(wg), dev(wu), dev(ids)
    act = empty_f32(k, ffn)
    qlin.call("qlin_launch_quant_swiglu_indexed_block", qtype, dg, du, eb, eb, rb, rb, dev(x), di, act, k, ffn, hid, 0)
    ref = orc.swiglu_indexed(qtype, wg, wu, eb, eb, rb, rb, x, ids, ffn, hid)
    assert normwise_rel_err(host(act), ref) <= 1e-4
    xq = orc.quantize_q8_1(x, hid)
    act8 = empty_f32(k, ffn)
    qlin.call("qlin_launch_quant_swiglu_indexed_q8_1", qtype, dg, du, eb, eb, rb, rb, dev(xq), di, act8, k, ffn, hid)
    got = host(act8)
    assert not got[2].any()
    assert normwise_rel_err(got, orc.swiglu_indexed_q8_1(qtype, wg, wu, eb, eb, rb, rb, xq, ids, ffn, hid)) <= 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("qtype,ffn", [(Q5_0, 1408), (Q8_0, 1408), (Q4_K, 1536), (Q6_K, 1536)])
def test_down_q8_1_and_f32_accum(qtype, ffn):
    """The routed down projections over Q8_1 act (plain and shared forms) and over f32 act, at C5's
    hidden size; routes are added in route order, so two calls give identical bits."""
    from gpu_util import banner, bind_stream, dev, host
    E, hid, k = 8, 2048, 6
    wd, rb, _ = qgen.random_matrix(qtype, E * hid, ffn, seed=60 + qtype)
    eb = hid * rb
    act = qgen.random_x(k, ffn, seed=61)
    aq = orc.quantize_q8_1(act, ffn)
    ids = np.array([1, 6, -1, 0, 6, 2], np.int32)
    rw = np.random.default_rng(62).random(k).astype(np.float32)
    out0 = np.random.default_rng(63).standard_normal(hid).astype(np.float32)
    banner(f"down q8_1 accum type={qtype} ffn={ffn}")
    bind_stream()
    dw, di, dr = dev(wd), dev(ids), dev(rw)
    ref = orc.down_q8_1_indexed_accum(qtype, wd, eb, rb, aq, ids, rw, out0, hid, ffn)
    results = []
    for name, a in (("qlin_launch_quant_down_q8_1_indexed_accum", dev(aq)),
                    ("qlin_launch_quant_down_q8_1_indexed_accum_shared", dev(aq)),
                    ("qlin_launch_quant_down_f32_indexed_accum", dev(act))):
        o = dev(out0)
        qlin.call(name, qtype, dw, eb, rb, a, di, dr, o, k, hid, ffn)
        got = host(o)
        assert normwise_rel_err(got - out0, ref - out0) <= 1e-5, name
        results.append(got)
    assert np.array_equal(results[0], results[1]) and np.array_equal(results[0], results[2])
