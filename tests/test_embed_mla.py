"""Quantized embedding lookup and MLA latent absorption (kernel.cu:2678-2693, 3004-3075, 3417-3453).

The reference has no tests of these kernels.  The oracle's sums are pinned on the CPU against numpy
restatements built from the independent encoder's values (tests/qgen.py) and a numpy decode of the
Q4_K min fields; the GPU tests compare the HIP kernels with the oracle at DeepSeek-V2-Lite's MLA
shapes (16 heads, qk_nope 128, qk_rope 64, v_head 128, kv_lora 512).
"""
import numpy as np
import pytest

import oracle as orc
import qgen
from blog_amd import qlin
from qgen import Q4_K, Q5_0, Q6_K, Q8_0, normwise_rel_err

TYPES = [Q4_K, Q6_K, Q5_0, Q8_0]
NH, QN, QR, VH, KL = 16, 128, 64, 128, 512          # DeepSeek-V2-Lite MLA


def q4k_min_coeffs(w: np.ndarray, rows: int, kv_lora: int) -> np.ndarray:
    """-dmin * m of every 32-block of every Q4_K row, decoded in numpy from the header bytes."""
    sb = w.reshape(rows, kv_lora // 256, 144)
    dmin = sb[:, :, 2:4].copy().view(np.float16)[..., 0].astype(np.float32)
    s = sb[:, :, 4:16].astype(np.int32)
    m = np.empty((rows, kv_lora // 256, 8), np.int32)
    m[:, :, :4] = s[:, :, 4:8] & 63
    m[:, :, 4:] = (s[:, :, 8:12] >> 4) | ((s[:, :, 4:8] >> 6) << 4)
    return -(dmin[:, :, None] * m.astype(np.float32)).reshape(rows, -1)


def kv_b(qtype, seed):
    return qgen.random_matrix(qtype, NH * (QN + VH), KL, seed=seed)


@pytest.mark.parametrize("qtype", TYPES)
def test_oracle_embedding_and_absorb_against_numpy(qtype):
    w, rb, vals = kv_b(qtype, 900 + qtype)
    ids = np.array([0, 5, 5, NH * (QN + VH) - 1], np.int32)
    assert np.array_equal(orc.quant_embedding(qtype, ids, w, rb, KL), vals[ids])
    rng = np.random.default_rng(qtype)
    q = rng.standard_normal(NH * (QN + QR)).astype(np.float32)
    W = vals.astype(np.float64).reshape(NH, QN + VH, KL)
    qh = q.astype(np.float64).reshape(NH, QN + QR)[:, :QN]
    ref = np.einsum("hdl,hd->hl", W[:, :QN], qh).reshape(-1)
    assert np.allclose(orc.mla_absorb_q_nope(qtype, q, w, rb, NH, QN, QR, VH, KL), ref, rtol=1e-12, atol=1e-12)
    latent = rng.standard_normal(NH * KL).astype(np.float32)
    ref_v = np.einsum("hvk,hk->hv", W[:, QN:], latent.astype(np.float64).reshape(NH, KL)).reshape(-1)
    delta = None
    if qtype == Q4_K:
        coeff = q4k_min_coeffs(w, NH * (QN + VH), KL).astype(np.float64).reshape(NH, QN + VH, -1)
        ref_d = np.einsum("hdb,hd->hb", coeff[:, :QN], qh).reshape(-1)
        got_d = orc.mla_absorb_q4_xsum_delta(q, w, rb, NH, QN, QR, VH, KL)
        assert np.allclose(got_d, ref_d, rtol=1e-12, atol=1e-12)
        delta = got_d.astype(np.float32)
        ref_v += np.einsum("hvb,hb->hv", coeff[:, QN:], delta.astype(np.float64).reshape(NH, -1)).reshape(-1)
    got_v = orc.mla_absorb_v(qtype, w, rb, latent, delta, NH, QN, VH, KL)
    assert np.allclose(got_v, ref_v, rtol=1e-12, atol=1e-12)


# ---- the HIP kernels ---------------------------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("qtype,hidden", [(Q4_K, 2048), (Q6_K, 2048), (Q5_0, 2048), (Q8_0, 896), (Q8_0, 32)])
def test_quant_embedding_bit_exact(qtype, hidden):
    from gpu_util import banner, bind_stream, dev, empty_f32, host
    vocab = 1000
    table, rb, _ = qgen.random_matrix(qtype, vocab, hidden, seed=hidden + qtype)
    ids = np.array([0, 999, 17, 17, 512, 3] * 3, np.int32)
    banner(f"embedding type={qtype} hidden={hidden}")
    bind_stream()
    out = empty_f32(len(ids), hidden)
    qlin.call("qlin_launch_quant_embedding", qtype, dev(ids), out, dev(table), rb, hidden, len(ids))
    got = host(out)
    ref = orc.quant_embedding(qtype, ids, table, rb, hidden)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("qtype", TYPES)
def test_mla_absorb_deepseek_shapes(qtype):
    from gpu_util import banner, bind_stream, dev, empty_f32, host
    w, rb, _ = kv_b(qtype, 910 + qtype)
    rng = np.random.default_rng(7 + qtype)
    q = rng.standard_normal(NH * (QN + QR)).astype(np.float32)
    latent = rng.standard_normal(NH * KL).astype(np.float32)
    banner(f"mla absorb type={qtype}")
    bind_stream()
    wd = dev(w)
    q_abs = empty_f32(NH * KL)
    qlin.call("qlin_launch_mla_absorb_q_nope", qtype, dev(q), wd, rb, q_abs, NH, QN, QR, VH, KL)
    ref = orc.mla_absorb_q_nope(qtype, q, w, rb, NH, QN, QR, VH, KL)
    assert normwise_rel_err(host(q_abs), ref) <= 1e-5
    delta_h, delta_d = None, None
    if qtype == Q4_K:
        nblk = KL // 32
        delta_d = empty_f32(NH * nblk)
        qlin.call("qlin_launch_mla_absorb_q4_xsum_delta", dev(q), wd, rb, delta_d, NH, QN, QR, VH, KL)
        ref_d = orc.mla_absorb_q4_xsum_delta(q, w, rb, NH, QN, QR, VH, KL)
        delta_h = host(delta_d)
        assert normwise_rel_err(delta_h, ref_d) <= 1e-5
    attn = empty_f32(NH * VH)
    qlin.call("qlin_launch_mla_absorb_v", qtype, wd, rb, dev(latent), delta_d, attn, NH, QN, VH, KL)
    ref_v = orc.mla_absorb_v(qtype, w, rb, latent, delta_h, NH, QN, VH, KL)
    assert normwise_rel_err(host(attn), ref_v) <= 1e-5
