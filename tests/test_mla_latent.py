"""MLA decode over the Q8_1 latent cache (kernel.cu:2945-3415, launch.cu:911-1049).

The reference has no tests of these kernels.  The oracle is pinned on the CPU: the store against the
Q8_1 quantizer (itself pinned by the reference's Q8_1 tests) and a numpy decode of its bytes; scores,
context and context_v against numpy restatements from a numpy decode of the cache; project_v against
the oracle's Q8_1 matmul (pinned against the reference's KATs) on the gathered rows and against a
float64 product of the dequantized operands.  The GPU tests compare the HIP kernels with the oracle at
DeepSeek-V2-Lite's MLA shapes (16 heads, qk_nope 128, qk_rope 64, v_head 128, kv_lora 512).
"""
import numpy as np
import pytest

import oracle as orc
import qgen
from blog_amd import qlin
from qgen import Q4_K, Q5_0, Q6_K, Q8_0, normwise_rel_err
from test_embed_mla import q4k_min_coeffs

NH, QN, QR, VH, KL = 16, 128, 64, 128, 512
SCALE = 1.0 / np.sqrt(QN + QR)


def decode_q8_1(cache, kv_lora):
    """(L [rows, kv_lora] float32, S - in-order block sums [rows, nb] float32) from Q8_1 rows."""
    rows, crb = cache.shape
    nb = (kv_lora + 31) // 32
    blk = cache[:, :nb * 36].reshape(rows, nb, 36)
    d = blk[:, :, 0:2].copy().view(np.float16)[..., 0].astype(np.float32)
    s = blk[:, :, 2:4].copy().view(np.float16)[..., 0].astype(np.float32)
    q = blk[:, :, 4:].view(np.int8).astype(np.float32)
    vals = d[:, :, None] * q                                  # exact in f32
    full = vals.reshape(rows, nb * 32)
    valid = (np.arange(nb * 32) < kv_lora).reshape(nb, 32)
    dsum = np.add.accumulate(np.where(valid, vals, 0.0).astype(np.float32), axis=2, dtype=np.float32)[:, :, -1]
    return full[:, :kv_lora], (s - dsum).astype(np.float32)


def make_cache(rows, kv_lora, qk_rope, seed, crb=None):
    """kv_cache f32 [rows, kv_lora + qk_rope] and its Q8_1 latent cache [rows, crb] (every row stored)."""
    rng = np.random.default_rng(seed)
    kv = rng.standard_normal((rows, kv_lora + qk_rope)).astype(np.float32)
    crb = crb or orc.q8_1_row_bytes(kv_lora)
    cache = np.zeros((rows, crb), np.uint8)
    for p in range(rows):
        cache = orc.mla_store_latent_q8_1(kv, cache, kv_lora, qk_rope, crb, p)
    return kv, cache, crb


def softmax64(s, pos):
    e = np.exp(s[:, :pos + 1].astype(np.float64) - s[:, :pos + 1].max(axis=1, keepdims=True))
    return e / (e.sum(axis=1, keepdims=True) + 1e-9)


# ---- the oracle, pinned on the CPU -----------------------------------------------------------------

@pytest.mark.parametrize("kv_lora,crb_extra", [(KL, 0), (500, 0), (KL, 36)])
def test_oracle_store_latent(kv_lora, crb_extra):
    rng = np.random.default_rng(kv_lora)
    kv = rng.standard_normal((5, kv_lora + QR)).astype(np.float32)
    crb = orc.q8_1_row_bytes(kv_lora) + crb_extra
    cache0 = rng.integers(0, 256, (5, crb), dtype=np.uint8)
    got = orc.mla_store_latent_q8_1(kv, cache0, kv_lora, QR, crb, 3)
    assert np.array_equal(np.delete(got, 3, 0), np.delete(cache0, 3, 0))   # only row pos changes
    nblk = crb // 36
    padded = np.zeros(nblk * 32, np.float32)
    padded[:kv_lora] = kv[3, :kv_lora]
    assert np.array_equal(got[3, :nblk * 36], orc.quantize_q8_1(padded, nblk * 32))
    L, _ = decode_q8_1(got[3:4], kv_lora)
    d = got[3, :nblk * 36].reshape(nblk, 36)[:, :2].copy().view(np.float16)[:, 0].astype(np.float32)
    # half a step of the f32 scale, plus 127 q-steps of its f16 rounding (2^-11 relative)
    assert np.all(np.abs(L[0] - kv[3, :kv_lora]) <= np.repeat(d, 32)[:kv_lora] * (0.5 + 127 * 2.0 ** -11) + 1e-7)
    if crb_extra:
        assert not got[3, (nblk - 1) * 36 + 4:nblk * 36].any()              # the padding block is zeros


def test_oracle_scores_context_against_numpy():
    T, pos = 40, 29
    kv, cache, crb = make_cache(T, KL, QR, 11)
    rng = np.random.default_rng(12)
    q_abs = rng.standard_normal((NH, KL)).astype(np.float32) * 0.1
    q = rng.standard_normal((NH, QN + QR)).astype(np.float32)
    delta = rng.standard_normal((NH, KL // 32)).astype(np.float32)
    L, C = decode_q8_1(cache, KL)
    ref = (q_abs.astype(np.float64) @ L.T.astype(np.float64) + q[:, QN:].astype(np.float64) @ kv[:, KL:].T
           + delta.astype(np.float64) @ C.T.astype(np.float64)) * np.float32(SCALE)
    got = orc.mla_absorb_scores(q_abs, q, cache, crb, delta, kv, NH, QN, QR, KL, pos, T, SCALE)
    assert np.allclose(got[:, :pos + 1], ref[:, :pos + 1], rtol=1e-9, atol=1e-9)
    assert np.isnan(got[:, pos + 1:]).all()                                  # positions past pos untouched
    # rope-only closed form
    zero = orc.mla_absorb_scores(np.zeros_like(q_abs), q, cache, crb, np.zeros_like(delta), kv, NH, QN, QR, KL,
                                 pos, T, SCALE)
    assert np.allclose(zero[:, :pos + 1], (q[:, QN:] @ kv[:pos + 1, KL:].T) * np.float32(SCALE), rtol=1e-5)

    s = rng.standard_normal((NH, T)).astype(np.float32) * 3
    lat, dl = orc.mla_absorb_context(s, cache, crb, NH, KL, pos, T)
    p = softmax64(s, pos)
    assert np.allclose(lat, p @ L[:pos + 1].astype(np.float64), rtol=1e-9, atol=1e-12)
    assert np.allclose(dl, p @ C[:pos + 1].astype(np.float64), rtol=1e-9, atol=1e-12)
    # identical rows: the weighted row is the row itself (the probabilities sum to 1 - 1e-9 / sum)
    same = np.repeat(cache[:1], T, 0)
    lat1, _ = orc.mla_absorb_context(s, same, crb, NH, KL, pos, T)
    assert np.allclose(lat1, np.broadcast_to(L[0], lat1.shape), rtol=1e-8, atol=1e-9)
    # pos beyond max_seq is clamped to the last position
    lat_c, _ = orc.mla_absorb_context(s, cache, crb, NH, KL, T + 5, T)
    assert np.allclose(lat_c, softmax64(s, T - 1) @ L.astype(np.float64), rtol=1e-9, atol=1e-12)


def test_oracle_attend_against_numpy():
    """The fused form: numpy scores, a softmax without the 1e-9 term, the weighted rows."""
    T, pos = 24, 17
    kv, cache, crb = make_cache(T, KL, QR, 13)
    rng = np.random.default_rng(14)
    q_abs = rng.standard_normal((NH, KL)).astype(np.float32) * 0.1
    q = rng.standard_normal((NH, QN + QR)).astype(np.float32)
    delta = rng.standard_normal((NH, KL // 32)).astype(np.float32)
    L, C = decode_q8_1(cache, KL)
    s = (q_abs.astype(np.float64) @ L.T.astype(np.float64) + q[:, QN:].astype(np.float64) @ kv[:, KL:].T
         + delta.astype(np.float64) @ C.T.astype(np.float64))[:, :pos + 1] * np.float32(SCALE)
    e = np.exp(s - s.max(axis=1, keepdims=True))
    p = e / e.sum(axis=1, keepdims=True)
    lat, dl = orc.mla_absorb_attend(q_abs, q, cache, crb, delta, kv, NH, QN, QR, KL, pos, T, SCALE)
    assert np.allclose(lat, p @ L[:pos + 1].astype(np.float64), rtol=1e-9, atol=1e-12)
    assert np.allclose(dl, p @ C[:pos + 1].astype(np.float64), rtol=1e-9, atol=1e-12)


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K, Q5_0, Q8_0])
def test_oracle_project_v(qtype):
    w, rb, vals = qgen.random_matrix(qtype, NH * (QN + VH), KL, seed=70 + qtype)
    kv, cache, crb = make_cache(4, KL, QR, 71)
    pos = 2
    kvb0 = np.random.default_rng(72).standard_normal((4, NH * (QN + VH)))
    got = orc.mla_project_v(qtype, w, rb, cache, crb, kvb0, NH, QN, VH, KL, pos)
    rows = np.array([h * (QN + VH) + QN + v for h in range(NH) for v in range(VH)])
    mask = np.zeros(kvb0.shape, bool)
    mask[pos, rows] = True
    assert np.array_equal(got[~mask], kvb0[~mask])
    w_rows = w.reshape(NH * (QN + VH), rb)[rows]
    assert np.array_equal(got[pos, rows], orc.matmul_q8_1(qtype, w_rows, rb, cache[pos], len(rows), KL, 1)[0])
    L, C = decode_q8_1(cache[pos:pos + 1], KL)
    ref = vals[rows].astype(np.float64) @ L[0].astype(np.float64)
    if qtype == Q4_K:
        # the min term uses the block's stored f16 sum: -dmin * m * (S - sum of L) on top of w . L
        ref += q4k_min_coeffs(w_rows, len(rows), KL).astype(np.float64) @ C[0].astype(np.float64)
    assert normwise_rel_err(got[pos, rows], ref) <= 1e-5


def test_oracle_context_v():
    T, pos = 33, 20
    rng = np.random.default_rng(80)
    s = rng.standard_normal((NH, T)).astype(np.float32)
    kvb = rng.standard_normal((T, NH * (QN + VH))).astype(np.float32)
    got = orc.mla_absorb_context_v(s, kvb, NH, QN, VH, pos, T)
    V = kvb.reshape(T, NH, QN + VH)[:, :, QN:].astype(np.float64)           # [T, h, v]
    ref = np.einsum("ht,thv->hv", softmax64(s, pos), V[:pos + 1])
    assert np.allclose(got, ref, rtol=1e-9, atol=1e-12)


# ---- the HIP kernels ---------------------------------------------------------------------------

def _pos(p):
    from gpu_util import dev
    return dev(np.array([p], np.int32))


@pytest.mark.gpu
@pytest.mark.parametrize("kv_lora,crb_extra", [(KL, 0), (500, 0), (KL, 36)])
def test_store_latent_bit_exact(kv_lora, crb_extra):
    from gpu_util import banner, bind_stream, dev, host
    rng = np.random.default_rng(90 + kv_lora)
    kv = rng.standard_normal((6, kv_lora + QR)).astype(np.float32)
    kv[2, :40] = 0.0                                                        # an all-zero block
    crb = orc.q8_1_row_bytes(kv_lora) + crb_extra
    cache0 = rng.integers(0, 256, (6, crb), dtype=np.uint8)
    banner(f"mla store latent kv_lora={kv_lora} crb={crb}")
    bind_stream()
    cd = dev(cache0)
    for p in (0, 2, 5):
        qlin.call("qlin_launch_mla_store_latent_q8_1_device_pos", dev(kv), cd, kv_lora, QR, crb, _pos(p))
    ref = cache0
    for p in (0, 2, 5):
        ref = orc.mla_store_latent_q8_1(kv, ref, kv_lora, QR, crb, p)
    assert np.array_equal(host(cd), ref)


@pytest.mark.gpu
@pytest.mark.parametrize("n_heads,T,pos", [(NH, 256, 0), (NH, 256, 37), (NH, 256, 255), (NH, 64, 100), (20, 48, 47)])
def test_scores_and_context(n_heads, T, pos):
    """Scores for t <= pos (entries past pos keep their contents), then the softmax context, at
    DeepSeek's MLA shape; pos past max_seq_len is clamped; 20 heads leave a partial head tile."""
    from gpu_util import banner, bind_stream, dev, empty_f32, host
    kv, cache, crb = make_cache(T, KL, QR, 100 + pos)
    rng = np.random.default_rng(101 + pos)
    q_abs = rng.standard_normal((n_heads, KL)).astype(np.float32) * 0.05
    q = rng.standard_normal((n_heads, QN + QR)).astype(np.float32) * 0.5
    delta = rng.standard_normal((n_heads, KL // 32)).astype(np.float32)
    banner(f"mla scores/context heads={n_heads} T={T} pos={pos}")
    bind_stream()
    s0 = np.full((n_heads, T), -7.0, np.float32)
    sd = dev(s0)
    cd, kd = dev(cache), dev(kv)
    qlin.call("qlin_launch_mla_absorb_scores_device_pos", dev(q_abs), dev(q), cd, crb, dev(delta), kd, sd, n_heads,
              QN, QR, KL, _pos(pos), T, SCALE)
    got = host(sd)
    ref = orc.mla_absorb_scores(q_abs, q, cache, crb, delta, kv, n_heads, QN, QR, KL, pos, T, SCALE)
    last = min(pos, T - 1)
    assert normwise_rel_err(got[:, :last + 1], ref[:, :last + 1]) <= 1e-5
    assert np.array_equal(got[:, last + 1:], s0[:, last + 1:])

    lat_d, dl_d = empty_f32(n_heads, KL), empty_f32(n_heads, KL // 32)
    qlin.call("qlin_launch_mla_absorb_context_device_pos", sd, cd, crb, dl_d, lat_d, n_heads, KL, _pos(pos), T)
    lat, dl = orc.mla_absorb_context(got, cache, crb, n_heads, KL, pos, T)
    assert normwise_rel_err(host(lat_d), lat) <= 1e-5
    assert normwise_rel_err(host(dl_d), dl) <= 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("T,pos", [(256, 0), (256, 255), (1024, 700)])
def test_attend_fused(T, pos):
    from gpu_util import banner, bind_stream, dev, empty_f32, host
    kv, cache, crb = make_cache(T, KL, QR, 130 + pos)
    rng = np.random.default_rng(131 + pos)
    q_abs = rng.standard_normal((NH, KL)).astype(np.float32) * 0.05
    q = rng.standard_normal((NH, QN + QR)).astype(np.float32) * 0.5
    delta = rng.standard_normal((NH, KL // 32)).astype(np.float32)
    banner(f"mla attend T={T} pos={pos}")
    bind_stream()
    lat_d, dl_d = empty_f32(NH, KL), empty_f32(NH, KL // 32)
    qlin.call("qlin_launch_mla_absorb_attend_device_pos", dev(q_abs), dev(q), dev(cache), crb, dev(delta), dl_d,
              dev(kv), lat_d, NH, QN, QR, KL, _pos(pos), T, SCALE)
    lat, dl = orc.mla_absorb_attend(q_abs, q, cache, crb, delta, kv, NH, QN, QR, KL, pos, T, SCALE)
    assert normwise_rel_err(host(lat_d), lat) <= 1e-5
    assert normwise_rel_err(host(dl_d), dl) <= 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("qtype", [Q4_K, Q6_K, Q5_0, Q8_0])
def test_project_v(qtype):
    from gpu_util import banner, bind_stream, dev, host
    w, rb, _ = qgen.random_matrix(qtype, NH * (QN + VH), KL, seed=110 + qtype)
    kv, cache, crb = make_cache(8, KL, QR, 111)
    kvb0 = np.random.default_rng(112).standard_normal((8, NH * (QN + VH))).astype(np.float32)
    banner(f"mla project_v type={qtype}")
    bind_stream()
    kd = dev(kvb0)
    qlin.call("qlin_launch_mla_project_v_device_pos", qtype, dev(w), rb, dev(cache), crb, kd, NH, QN, VH, KL, _pos(5))
    got = host(kd)
    ref = orc.mla_project_v(qtype, w, rb, cache, crb, kvb0, NH, QN, VH, KL, 5)
    rows = np.array([h * (QN + VH) + QN + v for h in range(NH) for v in range(VH)])
    assert normwise_rel_err(got[5, rows], ref[5, rows]) <= 1e-5
    keep = np.ones(kvb0.shape, bool)
    keep[5, rows] = False
    assert np.array_equal(got[keep], kvb0[keep])


@pytest.mark.gpu
@pytest.mark.parametrize("T,pos", [(256, 0), (256, 200), (4096, 4095)])
def test_context_v(T, pos):
    from gpu_util import banner, bind_stream, dev, empty_f32, host
    rng = np.random.default_rng(120 + pos)
    s = rng.standard_normal((NH, T)).astype(np.float32) * 2
    kvb = rng.standard_normal((T, NH * (QN + VH))).astype(np.float32)
    banner(f"mla context_v T={T} pos={pos}")
    bind_stream()
    out = empty_f32(NH, VH)
    qlin.call("qlin_launch_mla_absorb_context_v_device_pos", dev(s), dev(kvb), out, NH, QN, VH, _pos(pos), T)
    assert normwise_rel_err(host(out), orc.mla_absorb_context_v(s, kvb, NH, QN, VH, pos, T)) <= 1e-5
