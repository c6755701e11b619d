"""Parity of the HIP kernels (through the C ABI) with the CPU oracle on the same seeded inputs.

Bars: dequantized values bit-exact (f32 and f16); Q8_1 bytes bit-exact; router indices exact;
linear outputs within max|y - ref| / max|ref| <= 1e-3 (the gate).  Linear outputs must also be
fp32-accurate: max|y - ref| <= 2e-5 * max(|W| |x|), the error scale of an f32 dot product of
that conditioning (the Q4_K decode path multiplies on the matrix cores with x split into two bf16
parts, worst case about 1e-5 of sum|w x|).
"""
import numpy as np
import pytest
import torch

import oracle as orc
import qgen
from blog_amd import qlin
from gpu_util import banner, bind_stream, dev, empty_f32, host
from qgen import Q4_0, Q5_0, Q8_0, Q4_K, Q6_K, f16_bits, normwise_rel_err

pytestmark = pytest.mark.gpu

GATE = 1e-3
FP32 = 1e-5      # normwise fp32 deviation bound for the other entry points
COND = 2e-5      # max|y - ref| / max(|W| |x|) bound for the GEMV paths


def cond_err(y, ref, vals, x) -> float:
    """max|y - ref| relative to the largest sum_k |w_ik x_k| (the dot products' error scale)."""
    scale = np.abs(vals.astype(np.float64)) @ np.abs(np.asarray(x, np.float64).reshape(-1, vals.shape[1])).T
    return float(np.max(np.abs(np.asarray(y, np.float64).reshape(scale.T.shape) - np.asarray(ref).reshape(scale.T.shape)))
                 / np.max(scale))


@pytest.fixture(autouse=True)
def _stream():
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    bind_stream()
    yield
    torch.cuda.synchronize()


def gpu_gemv(qtype, w, rb, x, out_dim, in_dim, m=1, w_offset=0):
    wd = dev(np.concatenate([np.zeros(w_offset, np.uint8), w])) if w_offset else dev(w)
    xd = dev(np.ascontiguousarray(x, np.float32).reshape(m, in_dim))
    yd = empty_f32(m, out_dim)
    qlin.quant_gemv(qtype, wd.data_ptr() + w_offset, rb, xd, yd, out_dim, in_dim, m)
    return host(yd)


# ---- dequant -----------------------------------------------------------------------------------

def edge_blocks(qtype):
    """Blocks with extreme f16 scales: subnormal, max finite, negative, zero."""
    rng = np.random.default_rng(5)
    w, _ = qgen.random_blocks(qtype, 8, rng)
    bb = qgen.BLOCK[qtype][1]
    w = w.reshape(8, bb).copy()
    scales = [0x0001, 0x03FF, 0x7BFF, 0xBC00, 0x0000, 0x8001, 0x3555, 0xFBFF]
    for i, s in enumerate(scales):
        off = 208 if qtype == Q6_K else 0
        w[i, off:off + 2] = np.array([s & 0xFF, s >> 8], np.uint8)
        if qtype == Q4_K:
            w[i, 2:4] = np.array([scales[-1 - i] & 0xFF, scales[-1 - i] >> 8], np.uint8)
    return w.reshape(-1)


@pytest.mark.parametrize("qtype", [Q4_0, Q5_0, Q8_0, Q4_K, Q6_K])
def test_dequant_bit_exact(qtype):
    rng = np.random.default_rng(200 + qtype)
    nb = 6000 if qgen.BLOCK[qtype][0] == 32 else 1500
    w, _ = qgen.random_blocks(qtype, nb, rng)
    w = np.concatenate([w, edge_blocks(qtype)])
    n = (w.size // qgen.BLOCK[qtype][1]) * qgen.BLOCK[qtype][0]
    banner(f"dequant type={qtype} n={n}")
    wd = dev(w)
    o16 = torch.zeros(n, dtype=torch.int16, device="cuda")
    o32 = empty_f32(n)
    qlin.dequantize(qtype, wd, o16, n, f16=True)
    qlin.dequantize(qtype, wd, o32, n, f16=False)
    _same_bits(host(o32).view(np.uint32), orc.dequant_f32(qtype, w, n).view(np.uint32), "f32")
    _same_bits(host(o16).view(np.uint16), orc.dequant_f16(qtype, w, n), "f16")


def _same_bits(got, ref, what):
    bad = np.nonzero(got != ref)[0]
    if bad.size:
        i = bad[:8]
        pytest.fail(f"{what}: {bad.size} mismatches, first at {i.tolist()}: got {got[i].tolist()} "
                    f"expected {ref[i].tolist()}")


def test_dequant_reference_names():
    w = qgen.random_matrix(Q4_K, 4, 512, seed=3)[0]
    n = 4 * 512
    o = torch.zeros(n, dtype=torch.int16, device="cuda")
    qlin.call("qlin_launch_dequantize_q4k_to_f16", dev(w), o, n)
    assert np.array_equal(host(o).view(np.uint16), orc.dequant_f16(Q4_K, w, n))


# ---- GEMV --------------------------------------------------------------------------------------

GEMV_CASES = [
    (Q4_K, 1, 256), (Q4_K, 3, 512), (Q4_K, 17, 3584), (Q4_K, 4097, 8448),
    (Q4_K, 512, 3584), (Q4_K, 3584, 3584), (Q4_K, 18944, 3584), (Q4_K, 3584, 18944),
    (Q8_0, 4096, 4096), (Q8_0, 7, 96), (Q8_0, 4864, 896), (Q8_0, 33, 256), (Q8_0, 1000, 8448),
    (Q8_0, 896, 896), (Q8_0, 896, 4864), (Q8_0, 128, 128),
    (Q4_0, 18944, 3584), (Q4_0, 3584, 18944), (Q4_0, 5, 64), (Q4_0, 17, 256), (Q4_0, 300, 4608),
    (Q5_0, 2048, 1408), (Q5_0, 5, 64), (Q5_0, 300, 4096), (Q5_0, 33, 128), (Q5_0, 100, 18944),
    (Q6_K, 64, 512), (Q6_K, 257, 2048), (Q6_K, 16384, 2048), (Q6_K, 33, 768), (Q6_K, 100, 7168),
    # long K on the int8 form, whose row stride is then a multiple of 4 bytes (18944) or of 16 (14336)
    (Q6_K, 100, 18944), (Q6_K, 64, 14336),
]


@pytest.mark.parametrize("qtype,out_dim,in_dim", GEMV_CASES)
def test_gemv_parity(qtype, out_dim, in_dim):
    # block scales f16(|N(0,1)| * 0.01), and * 0.02 for Q4_0 as the Qwen2-7B Q4_0 FFN configuration draws them
    w, rb, vals = qgen.random_matrix(qtype, out_dim, in_dim, seed=out_dim * 7 + in_dim + qtype,
                                     scale=0.02 if qtype == Q4_0 else 0.01)
    x = qgen.random_x(1, in_dim, seed=in_dim + 1)
    banner(f"gemv type={qtype} N={out_dim} K={in_dim}")
    y = gpu_gemv(qtype, w, rb, x, out_dim, in_dim)
    ref = orc.matmul_f64(qtype, w, rb, x, out_dim, in_dim)
    err = normwise_rel_err(y, ref)
    assert err <= GATE, err
    assert cond_err(y, ref, vals, x) <= COND


@pytest.mark.parametrize("qtype,out_dim,in_dim", [(Q4_K, 300, 3584), (Q4_K, 1000, 8448), (Q8_0, 300, 4096),
                                                  (Q8_0, 300, 896), (Q4_0, 1000, 3584), (Q5_0, 300, 1408)])
def test_gemv_generic_path_agrees(qtype, out_dim, in_dim):
    """A weight pointer 2 bytes off the alignment the matrix-core kernel needs takes the generic
    kernel: both agree with the oracle."""
    w, rb, _ = qgen.random_matrix(qtype, out_dim, in_dim, seed=11)
    x = qgen.random_x(1, in_dim, seed=12)
    banner(f"gemv generic type={qtype} N={out_dim} K={in_dim}")
    y_fast = gpu_gemv(qtype, w, rb, x, out_dim, in_dim)
    y_gen = gpu_gemv(qtype, w, rb, x, out_dim, in_dim, w_offset=2)
    ref = orc.matmul_f64(qtype, w, rb, x, out_dim, in_dim)
    assert normwise_rel_err(y_fast, ref) <= FP32
    assert normwise_rel_err(y_gen, ref) <= FP32


@pytest.mark.parametrize("qtype,out_dim,in_dim", [(Q6_K, 300, 2048), (Q6_K, 70, 4096), (Q6_K, 64, 10240),
                                                  (Q4_0, 300, 3584),
                                                  (Q4_0, 33, 256), (Q8_0, 300, 4096), (Q8_0, 77, 1024)])
def test_rows_of_16_byte_units_and_offset_base(qtype, out_dim, in_dim):
    """Rows that are whole 16-byte units (Q4_0 always, Q8_0 with an even number of 128-weight chunks,
    Q6_K of 8k super-blocks), from a 16-byte aligned base and from one 4 bytes further.  Q6_K reads
    aligned 16-byte pieces from the first (the offsets of its super-blocks into a unit cycle through
    0..14) and dwords from the second.  Both agree with the oracle."""
    w, rb, vals = qgen.random_matrix(qtype, out_dim, in_dim, seed=out_dim + 3 * in_dim + qtype)
    assert rb % 16 == 0
    x = qgen.random_x(1, in_dim, seed=in_dim + 5)
    banner(f"gemv 16-byte units type={qtype} N={out_dim} K={in_dim}")
    ref = orc.matmul_f64(qtype, w, rb, x, out_dim, in_dim)
    for off in (0, 4):
        y = gpu_gemv(qtype, w, rb, x, out_dim, in_dim, w_offset=off)
        assert normwise_rel_err(y, ref) <= GATE
        assert cond_err(y, ref, vals, x) <= COND


@pytest.mark.parametrize("qtype,m", [(Q4_K, 2), (Q4_K, 5), (Q8_0, 3), (Q4_0, 9)])
def test_gemv_several_rows(qtype, m):
    in_dim = 1024
    w, rb, _ = qgen.random_matrix(qtype, 200, in_dim, seed=m)
    x = qgen.random_x(m, in_dim, seed=m + 1)
    banner(f"gemv m={m} type={qtype}")
    y = gpu_gemv(qtype, w, rb, x, 200, in_dim, m=m)
    ref = orc.matmul_f64(qtype, w, rb, x, 200, in_dim)
    assert normwise_rel_err(y, ref) <= FP32
    # the matmul entry point computes the same contraction
    yd = empty_f32(m, 200)
    qlin.quant_matmul(qtype, dev(w), rb, dev(x), yd, 200, in_dim, m)
    assert normwise_rel_err(host(yd), ref) <= FP32


@pytest.mark.parametrize("qtype,out_dim,in_dim,m", [
    (Q4_K, 200, 1024, 2), (Q4_K, 1000, 3584, 16), (Q4_K, 2816, 2048, 17), (Q4_K, 96, 256, 64), (Q4_K, 40, 4608, 65),
    (Q4_K, 33, 512, 130),
    (Q8_0, 4864, 896, 32), (Q8_0, 896, 4864, 32), (Q8_0, 50, 96, 5),     # C3's prompt: K 896 = 3.5 chunks
    (Q4_0, 300, 3584, 16), (Q5_0, 2048, 1408, 6), (Q6_K, 77, 2048, 20), (Q6_K, 77, 2048, 70),
    (Q6_K, 300, 512, 129)])
def test_matmul_rows_f32_matrix_cores(qtype, out_dim, in_dim, m):
    """m > 1 rows (launch_quant_matmul, kernel.cu:1254-1279) on the matrix cores: below 64 rows, Q4_K on
    the bf16 ones (x as bf16 hi + lo) and the other formats on the f32 ones; from 64 rows, Q4_K and Q6_K
    on the prefill GEMM (fp16, x as scaled hi + lo).  Row tails (out_dim % 16, and of the GEMM's 256-row
    tiles), fewer and more chunks than waves, a partial last chunk (K / 32 not a multiple of 8), token
    tails within and across 64-token tiles, and every format."""
    w, rb, vals = qgen.random_matrix(qtype, out_dim, in_dim, seed=out_dim + m + qtype)
    x = qgen.random_x(m, in_dim, seed=m + 7)
    banner(f"dense matmul type={qtype} n={out_dim} k={in_dim} m={m}")
    yd = empty_f32(m, out_dim)
    qlin.quant_matmul(qtype, dev(w), rb, dev(x), yd, out_dim, in_dim, m)
    y = host(yd)
    ref = orc.matmul_f64(qtype, w, rb, x, out_dim, in_dim)
    assert normwise_rel_err(y, ref) <= FP32
    assert cond_err(y, ref, vals, x) <= COND


@pytest.mark.parametrize("qtype,m", [(Q4_K, 16), (Q4_K, 1), (Q8_0, 3)])
def test_matmul_add_rows(qtype, m):
    """y[r] += W x[r] for a batch (the shared experts' down projection added into the MoE output,
    SharedExperts.cpp:42-48): each row equals the reference's gemv_add on that row."""
    out_dim, in_dim = 2048, 2816 if qtype == Q4_K else 512
    w, rb, _ = qgen.random_matrix(qtype, out_dim, in_dim, seed=41 + m)
    x = qgen.random_x(m, in_dim, seed=42 + m)
    y0 = np.random.default_rng(43).standard_normal((m, out_dim)).astype(np.float32) * 10
    yd = dev(y0)
    banner(f"matmul_add type={qtype} m={m}")
    qlin.quant_matmul_add(qtype, dev(w), rb, dev(x), yd, out_dim, in_dim, m)
    got = host(yd)
    for r in range(m):
        ref = orc.gemv_add(qtype, w, rb, x[r], y0[r], out_dim, in_dim)
        assert normwise_rel_err(got[r] - y0[r], ref - y0[r]) <= FP32


@pytest.mark.parametrize("qtype,ffn,hid,m", [(Q4_K, 2816, 2048, 16), (Q4_K, 200, 768, 5), (Q4_K, 200, 768, 1),
                                            (Q8_0, 96, 512, 3), (Q6_K, 2816, 2048, 16), (Q5_0, 100, 160, 4)])
def test_swiglu_rows(qtype, ffn, hid, m):
    """act[r] = silu(Wg x[r]) * (Wu x[r]) for a batch: C5's shared experts ([2816, 2048] Q4_K gate/up,
    16 tokens), a short batch, one row (the single-row kernel) and the other formats on the f32
    matrix-core kernel."""
    wg, rb, _ = qgen.random_matrix(qtype, ffn, hid, seed=ffn + m)
    wu, _, _ = qgen.random_matrix(qtype, ffn, hid, seed=ffn + m + 1)
    x = qgen.random_x(m, hid, seed=m + 3)
    act_d = empty_f32(m, ffn)
    banner(f"swiglu_rows type={qtype} ffn={ffn} m={m}")
    qlin.quant_swiglu_rows(qtype, dev(wg), dev(wu), rb, rb, dev(x), act_d, ffn, hid, m)
    got = host(act_d)
    for r in range(m):
        assert normwise_rel_err(got[r], orc.swiglu(qtype, wg, wu, rb, rb, x[r], ffn, hid)) <= 1e-4


@pytest.mark.parametrize("qtype", [Q4_K, Q8_0, Q5_0])
def test_gemv_add(qtype):
    in_dim = 512
    w, rb, _ = qgen.random_matrix(qtype, 333, in_dim, seed=21)
    x = qgen.random_x(1, in_dim, seed=22)[0]
    y0 = np.random.default_rng(23).standard_normal(333).astype(np.float32) * 100
    yd = dev(y0)
    banner(f"gemv_add type={qtype}")
    qlin.quant_gemv_add(qtype, dev(w), rb, dev(x), yd, 333, in_dim)
    ref = orc.gemv_add(qtype, w, rb, x, y0, 333, in_dim)
    assert normwise_rel_err(host(yd), ref) <= FP32


def test_q4k_wide_plans_take_the_vector_streaming_kernel():
    """[16448, 32768] Q4_K: the matrix-core kernel's LDS plan (x, 128 KB, plus 80 rows x 128 chunk
    partials) exceeds 160 KB, so the GEMV takes the VALU streaming kernel (qlin_q4k_stream.hip, x
    staged as f32, partials per 16 chunks).  The weight repeats a random [64, 32768] block, so every
    row's reference is one of 64 oracle dots."""
    n_unique, out_dim, in_dim = 64, 16448, 32768
    w, rb, _ = qgen.random_matrix(Q4_K, n_unique, in_dim, seed=77)
    x = qgen.random_x(1, in_dim, seed=78)
    ref = np.tile(orc.matmul_f64(Q4_K, w, rb, x, n_unique, in_dim)[0], out_dim // n_unique)
    banner(f"gemv vector streaming kernel N={out_dim} K={in_dim}")
    y = gpu_gemv(Q4_K, np.tile(w, out_dim // n_unique), rb, x, out_dim, in_dim)[0]
    assert normwise_rel_err(y, ref) <= FP32


def test_gemm_facade_derives_row_bytes():
    w, rb, _ = qgen.random_matrix(Q4_K, 96, 768, seed=31)
    x = qgen.random_x(1, 768, seed=32)
    yd = empty_f32(1, 96)
    qlin.call("qlin_gemm", Q4_K, dev(w), w.size, dev(x), yd, 96, 768, 1)
    assert normwise_rel_err(host(yd), orc.matmul_f64(Q4_K, w, rb, x, 96, 768)) <= FP32


def test_gemv_linearity_full_size():
    """Size-independent property at the metric's gate shape: y(a x1 + b x2) = a y(x1) + b y(x2)."""
    w, rb, _ = qgen.random_matrix(Q4_K, 18944, 3584, seed=41)
    x = qgen.random_x(2, 3584, seed=42)
    banner("gemv linearity 18944x3584")
    y = gpu_gemv(Q4_K, w, rb, x[0], 18944, 3584)[0], gpu_gemv(Q4_K, w, rb, x[1], 18944, 3584)[0]
    yc = gpu_gemv(Q4_K, w, rb, 2.0 * x[0] - 0.5 * x[1], 18944, 3584)[0]
    assert normwise_rel_err(yc, 2.0 * y[0].astype(np.float64) - 0.5 * y[1]) <= FP32


def test_empty_calls_are_noops():
    w, rb, _ = qgen.random_matrix(Q4_K, 4, 256, seed=1)
    yd = dev(np.full(4, 7.0, np.float32))
    qlin.quant_gemv(Q4_K, dev(w), rb, dev(np.zeros(256, np.float32)), yd, 0, 256, 1)
    qlin.quant_gemv(Q4_K, dev(w), rb, dev(np.zeros(256, np.float32)), yd, 4, 256, 0)
    assert np.all(host(yd) == 7.0)


# ---- reference known-answer tests on the GPU (LaunchAddTest.cpp) --------------------------------

def _kat_blocks():
    from test_oracle import kat_x, q4k_kat_block, q6k_kat_block
    return kat_x(), q4k_kat_block(), q6k_kat_block()


@pytest.mark.parametrize("which", ["q4k", "q6k"])
def test_kats(which):
    x, q4k, q6k = _kat_blocks()
    qtype, w, expected = (Q4_K, q4k, 2212.0) if which == "q4k" else (Q6_K, q6k, 948.0)
    y = gpu_gemv(qtype, w, w.size, x, 1, 256)
    assert abs(y[0, 0] - expected) <= 1e-3
    xq = torch.zeros(qlin.lib().qlin_q8_1_row_bytes(256), dtype=torch.uint8, device="cuda")
    qlin.quantize_q8_1(dev(x), xq, 256, 1)
    yd = empty_f32(1, 1)
    qlin.quant_matmul_q8_1(qtype, dev(w), w.size, xq, yd, 1, 256, 1)
    assert abs(host(yd)[0, 0] - expected) <= 1e-3


@pytest.mark.parametrize("which", ["q4k", "q6k"])
def test_kats_matrix_core_path(which):
    """The reference known answers through the matrix-core kernel: 16 rows of two KAT super-blocks
    (K = 512, whose row sizes meet that kernel's alignment), x = the KAT vector twice."""
    x, q4k, q6k = _kat_blocks()
    qtype, blk, expected = (Q4_K, q4k, 2212.0) if which == "q4k" else (Q6_K, q6k, 948.0)
    w = np.tile(blk, 2 * 16)
    y = gpu_gemv(qtype, w, 2 * blk.size, np.concatenate([x, x]), 16, 512)
    assert np.all(np.abs(y[0] - 2 * expected) <= 2e-3), y[0]


def test_kat_q8_0_rows_and_q8_1_sums():
    w = np.zeros(68, np.uint8)
    for row in range(2):
        w[row * 34:row * 34 + 2] = [0x00, 0x3C]
        for k in range(32):
            w[row * 34 + 2 + k] = (1 if row == 0 else (2 if k % 2 == 0 else -1)) & 0xFF
    x = np.array(list(range(1, 33)) + [-v for v in range(1, 33)] + [1, -1] * 16, np.float32).reshape(3, 32)
    yd = empty_f32(3, 2)
    qlin.quant_matmul(Q8_0, dev(w), 34, dev(x), yd, 2, 32, 3)
    y = host(yd)
    for r in range(3):
        assert abs(y[r, 0] - x[r].sum()) <= 1e-5
        assert abs(y[r, 1] - sum(x[r, k] * (2 if k % 2 == 0 else -1) for k in range(32))) <= 1e-5
    xs = np.full(32, 0.01, np.float32)
    xs[0] = 1.0
    for raw, expected in ((False, 158.0 / 127.0), (True, 1.31)):
        xq = torch.zeros(36, dtype=torch.uint8, device="cuda")
        qlin.quantize_q8_1(dev(xs), xq, 32, 1, store_raw_sum=raw)
        s = qgen.f16_val(host(xq)[2:4].view("<u2"))[0]
        assert abs(s - expected) <= 1e-3


# ---- Q8_1 ---------------------------------------------------------------------------------------

@pytest.mark.parametrize("raw", [False, True])
def test_quantize_q8_1_bit_exact(raw):
    in_dim, m = 4096 + 40, 5
    x = qgen.random_x(m, in_dim, seed=51) * np.float32(3.0)
    x[1, 64:96] = 0.0
    x[2, 5] = 1e-30
    rb = qlin.lib().qlin_q8_1_row_bytes(in_dim)
    xq = torch.zeros(m * rb, dtype=torch.uint8, device="cuda")
    qlin.quantize_q8_1(dev(x), xq, in_dim, m, store_raw_sum=raw)
    assert np.array_equal(host(xq), orc.quantize_q8_1(x, in_dim, raw))


@pytest.mark.parametrize("qtype,out_dim,in_dim,m", [(Q4_K, 96, 1024, 7), (Q6_K, 40, 512, 3), (Q8_0, 50, 256, 4),
                                                    (Q5_0, 33, 128, 2), (Q4_0, 17, 64, 3), (Q4_K, 512, 4096, 64),
                                                    (Q4_K, 300, 768, 70), (Q4_K, 257, 256, 1),
                                                    (Q4_K, 16, 512, 129),
                                                    # the 32-block formats' matrix-core GEMM: whole and
                                                    # partial 8-block units (K 1408 = 5.5 units, 192 =
                                                    # 0.75), row and token tails, one token
                                                    (Q8_0, 300, 4096, 70), (Q5_0, 2048, 1408, 96),
                                                    (Q4_0, 257, 192, 65), (Q8_0, 33, 64, 1), (Q5_0, 513, 2816, 17),
                                                    # Q6_K on the matrix cores (K a multiple of 512): both
                                                    # super-block parities, tails; K 768: per-element kernel
                                                    (Q6_K, 1000, 2048, 65), (Q6_K, 513, 512, 17), (Q6_K, 24, 768, 5),
                                                    # K / 32 odd: rows not 4-byte aligned, the per-element kernel
                                                    (Q8_0, 40, 96, 5), (Q5_0, 24, 160, 3),
                                                    # grids of at least half the CUs: the 8-wave, 64-token
                                                    # tiles (the cases above take the 4-wave, 32-token ones)
                                                    (Q4_0, 8192, 64, 256), (Q8_0, 4096, 128, 512)])
def test_matmul_q8_1_parity(qtype, out_dim, in_dim, m):
    w, rb, _ = qgen.random_matrix(qtype, out_dim, in_dim, seed=61 + out_dim)
    x = qgen.random_x(m, in_dim, seed=62)
    xq_h = orc.quantize_q8_1(x, in_dim)
    banner(f"matmul_q8_1 type={qtype} N={out_dim} K={in_dim} m={m}")
    yd = empty_f32(m, out_dim)
    qlin.quant_matmul_q8_1(qtype, dev(w), rb, dev(xq_h), yd, out_dim, in_dim, m)
    ref = orc.matmul_q8_1(qtype, w, rb, xq_h, out_dim, in_dim, m)
    assert normwise_rel_err(host(yd), ref) <= FP32


def test_q4k_gemm_c4_shape_every_row():
    """C4: Q4_K [14336, 4096] x Q8_1 activations [512, 4096] (f16 N(0,1) values) -> [512, 14336], every
    weight row checked against the oracle on 64 tokens: both ends of each of the 8 64-token tiles plus
    random ones, so every workgroup row and column of the grid is covered."""
    N, K, M = 14336, 4096, 512
    rng = np.random.default_rng(81)
    rb = K // 256 * 144
    w = rng.integers(0, 256, size=(N, K // 256, 144), dtype=np.uint8)
    w[:, :, 0:4] = f16_bits(np.abs(rng.standard_normal((N, K // 256, 2))) * 0.01).view(np.uint8).reshape(N, K // 256, 4)
    x = rng.standard_normal((M, K)).astype(np.float16).astype(np.float32)
    xq = orc.quantize_q8_1(x, K)
    banner("q4k gemm C4 shape 512x4096x14336")
    yd = empty_f32(M, N)
    qlin.quant_matmul_q8_1(Q4_K, dev(w.reshape(-1)), rb, dev(xq), yd, N, K, M)
    ends = np.array([[64 * t, 64 * t + 63] for t in range(M // 64)]).reshape(-1)
    rest = rng.choice(np.setdiff1d(np.arange(M), ends), 64 - ends.size, replace=False)
    toks = np.sort(np.concatenate([ends, rest]))
    assert toks.size == 64 and np.unique(toks).size == 64
    rbx = orc.q8_1_row_bytes(K)
    xq_t = np.ascontiguousarray(xq.reshape(M, rbx)[toks]).reshape(-1)
    ref = orc.matmul_q8_1(Q4_K, w.reshape(-1), rb, xq_t, N, K, toks.size, threads=0)
    assert normwise_rel_err(host(yd)[toks], ref) <= FP32
    # per row as well: no row may hide behind the others' norm
    got = host(yd)[toks]
    row_err = np.linalg.norm(got - ref, axis=0) / np.maximum(np.linalg.norm(ref, axis=0), 1e-30)
    assert row_err.max() <= 1e-5, (int(row_err.argmax()), float(row_err.max()))


def test_q6k_gemm_lm_head_shape_every_row():
    """DeepSeek-V2-Lite's lm_head in prefill: Q6_K [102400, 2048] x Q8_1 activations [512, 2048] -> [512,
    102400] (q6k_gemm_kernel, d applied once per super-block into output sums kept in LDS), every weight
    row checked against the oracle on 32 tokens: both ends of each of the 8 64-token tiles plus random
    ones, so every workgroup of the 3200 covers some checked outputs.  Random ql / qh / scale bytes, d =
    f16(|N(0,1)| * 0.01)."""
    N, K, M = 102400, 2048, 512
    rng = np.random.default_rng(83)
    rb = K // 256 * 210
    w = rng.integers(0, 256, size=(N, K // 256, 210), dtype=np.uint8)
    w[:, :, 208:210] = f16_bits(np.abs(rng.standard_normal((N, K // 256))) * 0.01).view(np.uint8).reshape(N, K // 256, 2)
    x = rng.standard_normal((M, K)).astype(np.float16).astype(np.float32)
    xq = orc.quantize_q8_1(x, K)
    banner("q6k gemm lm_head shape 512x2048x102400")
    yd = empty_f32(M, N)
    qlin.quant_matmul_q8_1(Q6_K, dev(w.reshape(-1)), rb, dev(xq), yd, N, K, M)
    ends = np.array([[64 * t, 64 * t + 63] for t in range(M // 64)]).reshape(-1)
    rest = rng.choice(np.setdiff1d(np.arange(M), ends), 32 - ends.size, replace=False)
    toks = np.sort(np.concatenate([ends, rest]))
    rbx = orc.q8_1_row_bytes(K)
    xq_t = np.ascontiguousarray(xq.reshape(M, rbx)[toks]).reshape(-1)
    ref = orc.matmul_q8_1(Q6_K, w.reshape(-1), rb, xq_t, N, K, toks.size, threads=0)
    got = host(yd)[toks]
    assert normwise_rel_err(got, ref) <= FP32
    row_err = np.linalg.norm(got - ref, axis=0) / np.maximum(np.linalg.norm(ref, axis=0), 1e-30)
    assert row_err.max() <= 1e-5, (int(row_err.argmax()), float(row_err.max()))


@pytest.mark.parametrize("qtype,N,K,M", [(Q4_K, 14336, 4096, 512), (Q6_K, 8192, 2048, 512),
                                         (Q4_K, 14336, 4096, 64), (Q6_K, 8192, 2048, 80)])
def test_f32_gemm_prefill_shape_every_row(qtype, N, K, M):
    """The engine's prefill entry (TensorTool::quant_direct_gemm -> launch_quant_matmul with f32
    activations, TensorTool.cpp:163-168, kernel.cu:1254-1279) on the fp16 matrix cores: Q4_K at
    Llama/Qwen-7B MLP shape [14336, 4096] and Q6_K at the DeepSeek-V2-Lite lm_head's K (2048, 8192 of
    its 102400 rows) x [M, K] N(0,1) f32 activations, every weight row checked against the f64
    oracle on 64 tokens that include both ends of every 64-token tile (every token when M <= 96).  At
    512 tokens the launch takes 256-row, 64-token workgroups; at 64 and 80 (a short prompt, more than
    half the CUs idle on those) 128-row, 32-token ones, 80 ending in half a token tile."""
    rng = np.random.default_rng(91 + qtype)
    bb = 144 if qtype == Q4_K else 210
    rb = K // 256 * bb
    w = rng.integers(0, 256, size=(N, K // 256, bb), dtype=np.uint8)
    if qtype == Q4_K:
        w[:, :, 0:4] = f16_bits(np.abs(rng.standard_normal((N, K // 256, 2))) * 0.01).view(np.uint8).reshape(N, K // 256, 4)
    else:
        w[:, :, 208:210] = f16_bits(np.abs(rng.standard_normal((N, K // 256, 1))) * 0.01).view(np.uint8).reshape(N, K // 256, 2)
    x = rng.standard_normal((M, K)).astype(np.float32)
    banner(f"f32 prefill gemm type={qtype} {M}x{K}x{N}")
    yd = empty_f32(M, N)
    qlin.quant_matmul(qtype, dev(w.reshape(-1)), rb, dev(x), yd, N, K, M)
    if M <= 96:
        toks = np.arange(M)
    else:
        ends = np.array([[64 * t, 64 * t + 63] for t in range(M // 64)]).reshape(-1)
        rest = rng.choice(np.setdiff1d(np.arange(M), ends), 64 - ends.size, replace=False)
        toks = np.sort(np.concatenate([ends, rest]))
    ref = orc.matmul_f64(qtype, w.reshape(-1), rb, x[toks], N, K)
    got = host(yd)[toks]
    assert normwise_rel_err(got, ref) <= FP32
    row_err = np.linalg.norm(got - ref, axis=0) / np.maximum(np.linalg.norm(ref, axis=0), 1e-30)
    assert row_err.max() <= 1e-5, (int(row_err.argmax()), float(row_err.max()))


@pytest.mark.parametrize("qtype", [Q4_K, Q6_K])
def test_f32_gemm_token_scales(qtype):
    """The prefill GEMM scales each token's 256 values of a super-block by a power of two into the
    fp16 range: tokens whose values span 1e-30 .. 1e30, an all-zero token, a token with one huge
    value among tiny ones and a super-block of zeros inside a token, each within 1e-5 of the f64
    oracle relative to that token's own largest output (a shared scale would lose the small ones)."""
    N, K, M = 300, 1024, 70
    w, rb, vals = qgen.random_matrix(qtype, N, K, seed=95)
    rng = np.random.default_rng(96)
    x = rng.standard_normal((M, K)).astype(np.float32)
    mags = [1e-30, 1e-12, 1e-3, 1.0, 1e3, 1e12, 1e30]
    for i in range(M):
        x[i] *= np.float32(mags[i % len(mags)])
    x[10] = 0.0
    x[11] = np.float32(1e-6) * rng.standard_normal(K).astype(np.float32)
    x[11, 77] = 1e6
    x[12, 256:512] = 0.0
    banner(f"f32 prefill gemm token scales type={qtype}")
    yd = empty_f32(M, N)
    qlin.quant_matmul(qtype, dev(w), rb, dev(x), yd, N, K, M)
    got = host(yd)
    ref = orc.matmul_f64(qtype, w, rb, x, N, K)
    assert np.all(got[10] == 0.0)
    for i in range(M):
        if i == 10:
            continue
        scale = np.max(np.abs(vals.astype(np.float64)) @ np.abs(x[i].astype(np.float64)))
        err = np.max(np.abs(got[i] - ref[i])) / scale
        assert err <= COND, (i, float(err))


@pytest.mark.parametrize("qtype,m", [(Q4_K, 64), (Q4_K, 96), (Q6_K, 96)])
def test_f32_gemm_add(qtype, m):
    """y += W x over m >= 64 tokens (launch_quant_matmul's add form) on the prefill GEMM."""
    N, K = 520, 2048
    w, rb, _ = qgen.random_matrix(qtype, N, K, seed=97 + m)
    x = qgen.random_x(m, K, seed=98 + m)
    y0 = np.random.default_rng(99).standard_normal((m, N)).astype(np.float32)
    banner(f"f32 prefill gemm add m={m}")
    yd = dev(y0)
    qlin.quant_matmul_add(qtype, dev(w), rb, dev(x), yd, N, K, m)
    ref = y0.astype(np.float64) + orc.matmul_f64(qtype, w, rb, x, N, K)
    assert normwise_rel_err(host(yd), ref) <= FP32


# ---- MoE ----------------------------------------------------------------------------------------

# up to 64 experts take the one-pass rank kernel, more the k-round argmax kernel
@pytest.mark.parametrize("ne,k", [(4, 6), (8, 6), (63, 6), (64, 6), (64, 8), (100, 6), (256, 6)])
def test_router_topk(ne, k):
    rng = np.random.default_rng(71 + ne + k)
    logits = rng.standard_normal((16, ne)).astype(np.float32)
    logits[3, :] = 0.5                                   # all tied: 0..k-1 in order
    logits[4, 7 % ne] = np.nan
    logits[5, :] = np.nan                                # nothing finite
    logits[6, [9 % ne, 4 % ne, ne - 4 if ne > 4 else 1]] = 9.0   # tie at the top
    logits[7, ne - 1] = np.inf                           # non-finite -> -inf
    logits[8, :] = -np.inf                               # two finite: the rest fall back to expert r
    logits[8, [ne - 1, ne // 2]] = [0.25, 0.75]
    logits[9, :] = rng.integers(-2, 3, ne).astype(np.float32)  # many ties
    scaling = 1.5
    idx_d = torch.zeros((16, k), dtype=torch.int32, device="cuda")
    w_d = empty_f32(16, k)
    qlin.call("qlin_launch_moe_router_topk", dev(logits), idx_d, w_d, 16, ne, k, scaling)
    idx_r, w_r = orc.router_topk(logits, k, scaling)
    assert np.array_equal(host(idx_d), idx_r)
    assert np.allclose(host(w_d), w_r, rtol=1e-5, atol=1e-7)


def _experts(qtype, E, rows, cols, seed):
    w, rb, vals = qgen.random_matrix(qtype, E * rows, cols, seed=seed)
    return w, rb, rows * rb


@pytest.mark.parametrize("n", [151936, 1000, 1])
def test_argmax(n):
    """Greedy pick over a Qwen2.5 vocabulary (launch_argmax, kernel.cu:3531-3592): ties go to the
    lowest index, NaN never wins, all -inf gives 0."""
    rng = np.random.default_rng(n)
    v = rng.standard_normal(n).astype(np.float32)
    banner(f"argmax n={n}")
    out = torch.empty(1, dtype=torch.int32, device="cuda")
    cases = [v]
    if n > 10:
        t = v.copy()
        t[[7, n - 3, n // 2]] = 50.0                 # a three-way tie
        nan = v.copy()
        nan[0] = np.nan
        cases += [t, nan, np.full(n, -np.inf, np.float32)]
    for c in cases:
        qlin.call("qlin_launch_argmax", dev(c), n, out)
        assert int(host(out)[0]) == orc.argmax(c)


def test_moe_accumulate_host_and_device_weight():
    e = np.random.default_rng(3).standard_normal(2048).astype(np.float32)
    o0 = np.random.default_rng(4).standard_normal(2048).astype(np.float32)
    banner("moe accumulate")
    o = dev(o0)
    qlin.call("qlin_launch_moe_accumulate", dev(e), 0.375, o, 2048)
    ref = o0 + np.float64(0.375) * e
    assert np.allclose(host(o), ref, rtol=0, atol=1e-6)
    qlin.call("qlin_launch_moe_accumulate_device", dev(e), dev(np.array([-2.0], np.float32)), o, 2048)
    assert np.allclose(host(o), ref - 2.0 * e, rtol=0, atol=1e-5)


def test_swiglu_indexed_and_down_ordered():
    E, ffn, hid, k = 8, 96, 512, 4
    wg, grb, geb = _experts(Q4_K, E, ffn, hid, 81)
    wu, _, _ = _experts(Q4_K, E, ffn, hid, 82)
    wdn, drb, deb = _experts(Q5_0, E, hid, ffn, 83)
    x = qgen.random_x(1, hid, seed=84)[0]
    ids = np.array([5, -1, 0, 7], np.int32)
    rw = np.array([0.4, 0.3, 0.2, 0.1], np.float32)
    act_d = empty_f32(k, ffn)
    qlin.call("qlin_launch_quant_swiglu_indexed", Q4_K, dev(wg), dev(wu), geb, geb, grb, grb, dev(x), dev(ids),
              act_d, k, ffn, hid)
    act_ref = orc.swiglu_indexed(Q4_K, wg, wu, geb, geb, grb, grb, x, ids, ffn, hid)
    act = host(act_d)
    assert np.all(act[1] == 0.0)
    assert normwise_rel_err(act, act_ref) <= 1e-4
    out0 = np.random.default_rng(85).standard_normal(hid).astype(np.float32)
    out_d = dev(out0)
    qlin.call("qlin_launch_quant_down_f32_indexed_accum_ordered", Q5_0, dev(wdn), deb, drb, dev(act_ref), dev(ids),
              dev(rw), out_d, k, hid, ffn)
    ref = orc.down_indexed_ordered(Q5_0, wdn, deb, drb, act_ref, ids, rw, out0, hid, ffn)
    assert normwise_rel_err(host(out_d), ref) <= FP32


ROUTED_CASES = [
    # DeepSeek-V2-Lite's routes (64 x [1408, 2048] Q4_K gate/up, [2048, 1408] Q5_0 down)
    (Q4_K, Q5_0, 64, 1408, 2048, [3, 17, 63, 0, 42, 9]),
    # tiles of 16 concatenated rows that span two routes (ffn 200, SwiGLU only), no expert, a repeat
    (Q4_K, Q8_0, 16, 200, 768, [5, -1, 5, 2]),
    (Q4_K, Q8_0, 16, 256, 768, [5, -1, 5, 2]),
    # 16 routes (the most one launch takes), Q6_K gate/up, Q4_K down
    (Q6_K, Q4_K, 8, 256, 512, [7, 1, -1, 0, 3, 2, 6, 4, 5, 1, 0, 2, 3, 4, 5, 6]),
    (Q4_K, Q6_K, 4, 512, 256, [-1, -1]),                 # no expert at all
    (Q8_0, Q5_0, 6, 384, 1024, [2, 4, 1]),
    (Q4_0, Q8_0, 5, 128, 256, [4, 0, 3, 1, 2, 4, 0, 3, 1, 2, 4, 0, 3, 1, 2, 4, 0]),  # 17 routes: per-element kernels
]


@pytest.mark.parametrize("gu_type,dn_type,E,ffn,hid,ids", ROUTED_CASES)
def test_routed_swiglu_and_down(gu_type, dn_type, E, ffn, hid, ids):
    """launch_quant_swiglu_indexed and launch_quant_down_f32_indexed_accum_ordered (kernel.cu:1340-1385,
    2253-2287) on the matrix-core routed forms, and from a base 2 bytes off their alignment on the
    per-element kernels: both agree with the oracle, and a route without an expert gives 0."""
    k = len(ids)
    ids = np.array(ids, np.int32)
    wg, grb, geb = _experts(gu_type, E, ffn, hid, 900 + ffn + k)
    wu, _, _ = _experts(gu_type, E, ffn, hid, 901 + ffn + k)
    # (a SwiGLU width that is not whole 32-weight blocks has no down projection)
    has_down = ffn % qgen.BLOCK[dn_type][0] == 0
    wdn, drb, deb = _experts(dn_type, E, hid, ffn, 902 + ffn + k) if has_down else (np.zeros(4, np.uint8), 0, 0)
    x = qgen.random_x(1, hid, seed=903 + k)[0]
    rw = np.random.default_rng(904 + k).uniform(0.05, 1.0, k).astype(np.float32)
    act_ref = orc.swiglu_indexed(gu_type, wg, wu, geb, geb, grb, grb, x, ids, ffn, hid)
    out0 = np.random.default_rng(905).standard_normal(hid).astype(np.float32)
    ref = orc.down_indexed_ordered(dn_type, wdn, deb, drb, act_ref, ids, rw, out0, hid, ffn) if has_down else None
    for off in (0, 2):
        banner(f"routed swiglu/down gu={gu_type} dn={dn_type} ffn={ffn} hid={hid} k={k} offset={off}")
        pad = np.zeros(off, np.uint8)
        wgd, wud, wdd = dev(np.concatenate([pad, wg])), dev(np.concatenate([pad, wu])), dev(np.concatenate([pad, wdn]))
        act_d = empty_f32(k, ffn)
        qlin.call("qlin_launch_quant_swiglu_indexed", gu_type, wgd.data_ptr() + off, wud.data_ptr() + off, geb, geb,
                  grb, grb, dev(x), dev(ids), act_d, k, ffn, hid)
        act = host(act_d)
        assert np.all(act[ids < 0] == 0.0)
        assert normwise_rel_err(act, act_ref) <= 1e-4
        if not has_down:
            continue
        out_d = dev(out0)
        qlin.call("qlin_launch_quant_down_f32_indexed_accum_ordered", dn_type, wdd.data_ptr() + off, deb, drb,
                  dev(act_ref), dev(ids), dev(rw), out_d, k, hid, ffn)
        got = host(out_d)
        if np.all(ids < 0):
            assert np.array_equal(got, out0)  # nothing added
            continue
        assert normwise_rel_err(got - out0, ref - out0) <= 1e-4
        assert normwise_rel_err(got, ref) <= FP32


def test_shared_swiglu():
    ffn, hid = 200, 768
    wg, rb, _ = qgen.random_matrix(Q4_K, ffn, hid, seed=91)
    wu, _, _ = qgen.random_matrix(Q4_K, ffn, hid, seed=92)
    x = qgen.random_x(1, hid, seed=93)[0]
    act_d = empty_f32(ffn)
    qlin.call("qlin_launch_quant_swiglu", Q4_K, dev(wg), dev(wu), rb, rb, dev(x), act_d, ffn, hid)
    assert normwise_rel_err(host(act_d), orc.swiglu(Q4_K, wg, wu, rb, rb, x, ffn, hid)) <= 1e-4


def test_moe_facade_deepseek_shape():
    """DeepSeek-V2-Lite routed experts (64 x [1408, 2048] Q4_K gate/up, [2048, 1408] Q5_0 down), k = 6."""
    E, ffn, hid, k = 64, 1408, 2048, 6
    wg, grb, geb = _experts(Q4_K, E, ffn, hid, 101)
    wu, _, _ = _experts(Q4_K, E, ffn, hid, 102)
    wdn, drb, deb = _experts(Q5_0, E, hid, ffn, 103)
    x = qgen.random_x(1, hid, seed=104)[0]
    logits = np.random.default_rng(105).standard_normal((1, E)).astype(np.float32)
    ids, rw = orc.router_topk(logits, k, 1.0)
    ids, rw = ids[0], rw[0]
    out0 = np.zeros(hid, np.float32)
    out_d = dev(out0)
    act_d = empty_f32(k, ffn)
    banner("moe facade deepseek shape")
    qlin.call("qlin_moe_routed_decode_indexed", Q4_K, dev(wg), dev(wu), wg.size, Q5_0, dev(wdn), wdn.size, E, ffn,
              hid, hid, dev(x), dev(ids), dev(rw), act_d, out_d, k)
    act_ref = orc.swiglu_indexed(Q4_K, wg, wu, geb, geb, grb, grb, x, ids, ffn, hid)
    ref = orc.down_indexed_ordered(Q5_0, wdn, deb, drb, act_ref, ids, rw, out0, hid, ffn)
    assert normwise_rel_err(host(out_d), ref) <= 1e-4


@pytest.mark.parametrize("E,k,ffn,hid,special", [(64, 6, 1408, 2048, None), (64, 6, 256, 512, "ties"),
                                                (48, 4, 256, 512, "nan"), (8, 6, 256, 256, "two_finite"),
                                                (100, 6, 256, 256, None)])
def test_moe_facade_from_router_logits(E, k, ffn, hid, special):
    """The router and the per-token routed decode in one call: up to 64 experts the routed gate/up
    launch picks the routes itself.  Its ids are the router's exactly, its weights the router's, and
    the output the indexed path's reference."""
    wg, grb, geb = _experts(Q4_K, E, ffn, hid, 111 + E)
    wu, _, _ = _experts(Q4_K, E, ffn, hid, 112 + E)
    wdn, drb, deb = _experts(Q5_0, E, hid, ffn, 113 + E)
    x = qgen.random_x(1, hid, seed=114)[0]
    rng = np.random.default_rng(115 + k)
    logits = rng.standard_normal((1, E)).astype(np.float32)
    if special == "ties":
        logits[0, :] = rng.integers(-1, 2, E).astype(np.float32)
    elif special == "nan":
        logits[0, [3, 7]] = [np.nan, np.inf]
    elif special == "two_finite":
        logits[0, :] = -np.inf
        logits[0, [E - 1, 2]] = [0.5, 0.25]
    ids_r, rw_r = orc.router_topk(logits, k, 0.75)
    ids_r, rw_r = ids_r[0], rw_r[0]
    out0 = np.random.default_rng(116).standard_normal(hid).astype(np.float32)
    out_d = dev(out0)
    act_d = empty_f32(k, ffn)
    ids_d = torch.full((k,), -5, dtype=torch.int32, device="cuda")
    rw_d = empty_f32(k)
    banner(f"moe facade from logits E={E} k={k} {special}")
    qlin.call("qlin_moe_routed_decode_indexed_logits", Q4_K, dev(wg), dev(wu), wg.size, Q5_0, dev(wdn), wdn.size, E,
              ffn, hid, hid, dev(x), dev(logits), 0.75, ids_d, rw_d, act_d, out_d, k)
    assert np.array_equal(host(ids_d), ids_r)
    assert np.allclose(host(rw_d), rw_r, rtol=1e-5, atol=1e-7)
    act_ref = orc.swiglu_indexed(Q4_K, wg, wu, geb, geb, grb, grb, x, ids_r, ffn, hid)
    ref = orc.down_indexed_ordered(Q5_0, wdn, deb, drb, act_ref, ids_r, host(rw_d), out0, hid, ffn)
    assert normwise_rel_err(host(out_d) - out0, ref - out0) <= 1e-4


def _moe_batch(gu_type, dn_type, E, ffn, hid, tokens, k, seed):
    wg, grb, geb = _experts(gu_type, E, ffn, hid, seed)
    wu, _, _ = _experts(gu_type, E, ffn, hid, seed + 1)
    wdn, drb, deb = _experts(dn_type, E, hid, ffn, seed + 2)
    rng = np.random.default_rng(seed + 3)
    x = rng.standard_normal((tokens, hid)).astype(np.float32)
    logits = rng.standard_normal((tokens, E)).astype(np.float32)
    ids, rw = orc.router_topk(logits, k, 1.0)
    return wg, wu, grb, geb, wdn, drb, deb, x, np.ascontiguousarray(ids), np.ascontiguousarray(rw)


def _moe_batch_ref(gu_type, dn_type, wg, wu, grb, geb, wdn, drb, deb, x, ids, rw, out0, ffn, hid):
    ref = out0.copy()
    for t in range(x.shape[0]):
        act = orc.swiglu_indexed(gu_type, wg, wu, geb, geb, grb, grb, x[t], ids[t], ffn, hid)
        ref[t] = orc.down_indexed_ordered(dn_type, wdn, deb, drb, act, ids[t], rw[t], ref[t], hid, ffn)
    return ref


def _run_grouped(gu_type, dn_type, wg, wu, wdn, E, ffn, hid, x, ids, rw, out0):
    tokens, k = ids.shape
    nbytes = qlin.lib().qlin_moe_grouped_workspace_bytes(tokens, k, E, ffn, hid)
    ws = torch.empty(nbytes + 256, dtype=torch.uint8, device="cuda")
    wsp = (ws.data_ptr() + 255) // 256 * 256
    out_d = dev(out0)
    qlin.call("qlin_moe_routed_decode_grouped", gu_type, dev(wg), dev(wu), wg.size, dn_type, dev(wdn), wdn.size, E,
              ffn, hid, hid, dev(x), dev(ids), dev(rw), wsp, nbytes, out_d, tokens, k)
    return host(out_d)


@pytest.mark.parametrize("dn_type", [Q5_0, Q8_0])
def test_moe_grouped_c5(dn_type):
    """C5: DeepSeek-V2-Lite routed experts for a batch of 16 tokens (64 x [1408, 2048] Q4_K gate/up,
    [2048, 1408] down, top-6) -- equal to the per-token reference path on every token."""
    E, ffn, hid, tokens, k = 64, 1408, 2048, 16, 6
    wg, wu, grb, geb, wdn, drb, deb, x, ids, rw = _moe_batch(Q4_K, dn_type, E, ffn, hid, tokens, k, 201)
    ids[3, 2] = -1                  # an empty route
    ids[5, :] = ids[4, :]           # two tokens with the same experts
    out0 = np.random.default_rng(7).standard_normal((tokens, hid)).astype(np.float32)
    banner(f"moe grouped C5 down={dn_type}")
    got = _run_grouped(Q4_K, dn_type, wg, wu, wdn, E, ffn, hid, x, ids, rw, out0)
    ref = _moe_batch_ref(Q4_K, dn_type, wg, wu, grb, geb, wdn, drb, deb, x, ids, rw, out0, ffn, hid)
    assert normwise_rel_err(got - out0, ref - out0) <= 1e-4
    assert normwise_rel_err(got, ref) <= 1e-5


@pytest.mark.parametrize("gu_type,dn_type,ffn", [(Q4_K, Q8_0, 128), (Q4_K, Q5_0, 256), (Q4_K, Q5_0, 96),
                                                  (Q6_K, Q8_0, 128), (Q4_K, Q4_K, 512)])
def test_moe_grouped_many_routes_per_expert_and_fallback(gu_type, dn_type, ffn):
    """Routes beyond one pass per expert (8 experts, 24 tokens x 4 routes, about 12 per expert), most
    workgroups without a tile, a down width that is not a multiple of 128 (96: the per-element down
    kernel), and Q6_K gate/up, which takes the per-token kernels inside the same entry point."""
    E, hid, tokens, k = 8, 512, 24, 4
    seed = 301 + ffn + 10 * dn_type + gu_type
    wg, wu, grb, geb, wdn, drb, deb, x, ids, rw = _moe_batch(gu_type, dn_type, E, ffn, hid, tokens, k, seed)
    out0 = np.zeros((tokens, hid), np.float32)
    banner(f"moe grouped passes gu={gu_type} dn={dn_type} ffn={ffn}")
    got = _run_grouped(gu_type, dn_type, wg, wu, wdn, E, ffn, hid, x, ids, rw, out0)
    ref = _moe_batch_ref(gu_type, dn_type, wg, wu, grb, geb, wdn, drb, deb, x, ids, rw, out0, ffn, hid)
    assert normwise_rel_err(got, ref) <= 1e-4


def test_moe_grouped_shared_experts_as_one_expert():
    """C5's 2 shared experts (SharedExperts.cpp:21-49: swiglu over the concatenated [2816, 2048] Q4_K
    gate/up, then a Q4_K [2048, 2816] down added into the MoE output) for 16 tokens, run as one
    expert that every token takes with weight 1.0, on top of an output that already holds the routed
    sum: the Q4_K streaming down kernel, 4 passes of 4 routes."""
    E, ffn, hid, tokens, k = 1, 2816, 2048, 16, 1
    wg, wu, grb, geb, wdn, drb, deb, x, _, _ = _moe_batch(Q4_K, Q4_K, E, ffn, hid, tokens, k, 351)
    ids = np.zeros((tokens, 1), np.int32)
    rw = np.ones((tokens, 1), np.float32)
    out0 = np.random.default_rng(9).standard_normal((tokens, hid)).astype(np.float32)
    banner("moe grouped shared experts")
    got = _run_grouped(Q4_K, Q4_K, wg, wu, wdn, E, ffn, hid, x, ids, rw, out0)
    ref = _moe_batch_ref(Q4_K, Q4_K, wg, wu, grb, geb, wdn, drb, deb, x, ids, rw, out0, ffn, hid)
    assert normwise_rel_err(got - out0, ref - out0) <= 1e-4
    # the reference's own two launches for one token: fused SwiGLU, then gemv_add into the output
    act = orc.swiglu(Q4_K, wg, wu, grb, grb, x[0], ffn, hid)
    ref0 = orc.gemv_add(Q4_K, wdn, drb, act, out0[0], hid, ffn)
    assert normwise_rel_err(got[0] - out0[0], ref0 - out0[0]) <= 1e-4


def test_moe_grouped_skewed_routing():
    """One expert chosen by every token (200 routes: 50 passes) beside 15 light ones: the workgroups
    split the tiles by cost, so the light experts' tiles pack densely and are taken in several LDS
    pieces per workgroup."""
    E, ffn, hid, tokens, k = 16, 1024, 512, 200, 2
    wg, wu, grb, geb, wdn, drb, deb, x, ids, rw = _moe_batch(Q4_K, Q5_0, E, ffn, hid, tokens, k, 341)
    ids = np.ascontiguousarray(np.stack([np.zeros(tokens, np.int32), 1 + np.arange(tokens, dtype=np.int32) % 15], 1))
    out0 = np.zeros((tokens, hid), np.float32)
    banner("moe grouped skewed routing")
    got = _run_grouped(Q4_K, Q5_0, wg, wu, wdn, E, ffn, hid, x, ids, rw, out0)
    ref = _moe_batch_ref(Q4_K, Q5_0, wg, wu, grb, geb, wdn, drb, deb, x, ids, rw, out0, ffn, hid)
    assert normwise_rel_err(got, ref) <= 1e-4


@pytest.mark.parametrize("E,tokens,k", [(300, 40, 4), (64, 300, 4)])
def test_moe_grouped_beyond_in_kernel_grouping(E, tokens, k):
    """More experts (300) or routes (1200) than the gate/up launch groups in its own LDS: the separate
    grouping launch writes the groups, and the streaming launches read them."""
    ffn, hid = 256, 256
    wg, wu, grb, geb, wdn, drb, deb, x, ids, rw = _moe_batch(Q4_K, Q5_0, E, ffn, hid, tokens, k, 361 + E)
    ids[1, 0] = -1
    out0 = np.zeros((tokens, hid), np.float32)
    banner(f"moe grouped beyond in-kernel grouping E={E} R={tokens * k}")
    got = _run_grouped(Q4_K, Q5_0, wg, wu, wdn, E, ffn, hid, x, ids, rw, out0)
    ref = _moe_batch_ref(Q4_K, Q5_0, wg, wu, grb, geb, wdn, drb, deb, x, ids, rw, out0, ffn, hid)
    assert normwise_rel_err(got, ref) <= 1e-4


@pytest.mark.parametrize("E,tokens,k,ffn,hid", [(64, 16, 6, 1408, 2048), (8, 24, 4, 256, 512), (100, 16, 6, 256, 256),
                                                (64, 300, 4, 256, 256)])
def test_moe_grouped_from_router_logits(E, tokens, k, ffn, hid):
    """The router and the batched decode in one call: up to 64 experts (and 1024 routes) the gate/up
    launch picks the routes itself.  Its ids are the router's exactly (ties, NaN, +inf, rows with only
    two finite logits), its weights the router's, and the output the per-token reference's."""
    wg, wu, grb, geb, wdn, drb, deb, x, _, _ = _moe_batch(Q4_K, Q5_0, E, ffn, hid, tokens, k, 381 + E + tokens)
    rng = np.random.default_rng(391 + E)
    logits = rng.standard_normal((tokens, E)).astype(np.float32)
    logits[1, :] = 0.5
    logits[2, 3] = np.nan
    logits[3, :] = -np.inf
    logits[3, [E - 1, E // 2]] = [0.25, 0.75]
    logits[4, E - 2] = np.inf
    logits[5, :] = rng.integers(-2, 3, E).astype(np.float32)
    ids_r, rw_r = orc.router_topk(logits, k, 1.25)
    nbytes = qlin.lib().qlin_moe_grouped_workspace_bytes(tokens, k, E, ffn, hid)
    ws = torch.empty(nbytes + 256, dtype=torch.uint8, device="cuda")
    wsp = (ws.data_ptr() + 255) // 256 * 256
    out0 = np.random.default_rng(13).standard_normal((tokens, hid)).astype(np.float32)
    out_d = dev(out0)
    ids_d = torch.full((tokens, k), -7, dtype=torch.int32, device="cuda")
    rw_d = empty_f32(tokens, k)
    banner(f"moe grouped from logits E={E} tokens={tokens} k={k}")
    qlin.call("qlin_moe_routed_decode_grouped_logits", Q4_K, dev(wg), dev(wu), wg.size, Q5_0, dev(wdn), wdn.size, E,
              ffn, hid, hid, dev(x), dev(logits), 1.25, ids_d, rw_d, wsp, nbytes, out_d, tokens, k)
    assert np.array_equal(host(ids_d), ids_r)
    assert np.allclose(host(rw_d), rw_r, rtol=1e-5, atol=1e-7)
    ref = _moe_batch_ref(Q4_K, Q5_0, wg, wu, grb, geb, wdn, drb, deb, x, ids_r, host(rw_d), out0, ffn, hid)
    assert normwise_rel_err(host(out_d) - out0, ref - out0) <= 1e-4


def test_moe_grouped_unaligned_output():
    """An output 4 bytes past a 16-byte boundary."""
    E, ffn, hid, tokens, k = 8, 256, 256, 4, 2
    wg, wu, grb, geb, wdn, drb, deb, x, ids, rw = _moe_batch(Q4_K, Q5_0, E, ffn, hid, tokens, k, 371)
    ids[2, 1] = -1
    out0 = np.random.default_rng(11).standard_normal((tokens, hid)).astype(np.float32)
    nbytes = qlin.lib().qlin_moe_grouped_workspace_bytes(tokens, k, E, ffn, hid)
    ws = torch.empty(nbytes + 256, dtype=torch.uint8, device="cuda")
    wsp = (ws.data_ptr() + 255) // 256 * 256
    buf = dev(np.concatenate([np.zeros(1, np.float32), out0.ravel()]))
    out_d = buf[1:]
    assert out_d.data_ptr() % 16 == 4
    banner("moe grouped unaligned output")
    qlin.call("qlin_moe_routed_decode_grouped", Q4_K, dev(wg), dev(wu), wg.size, Q5_0, dev(wdn), wdn.size, E,
              ffn, hid, hid, dev(x), dev(ids), dev(rw), wsp, nbytes, out_d, tokens, k)
    ref = _moe_batch_ref(Q4_K, Q5_0, wg, wu, grb, geb, wdn, drb, deb, x, ids, rw, out0, ffn, hid)
    assert normwise_rel_err(host(out_d).reshape(tokens, hid) - out0, ref - out0) <= 1e-4


@pytest.mark.parametrize("gu,E,tokens,k,ffn,hid,sffn,stype", [
    (Q4_K, 64, 16, 6, 1408, 2048, 2816, Q4_K),  # C5: the shared down-add applies the routed sum
    (Q4_K, 8, 5, 2, 256, 512, 512, Q4_K),       # a short batch, same form
    (Q4_K, 8, 6, 2, 256, 512, 160, Q8_0),       # shared Q8_0 (f32-element matrix-core kernel), same form
    (Q4_K, 8, 1, 2, 256, 512, 512, Q4_K),       # one token: the shared down-add is the decode GEMV, own combine
    (Q6_K, 8, 4, 2, 256, 512, 512, Q4_K),       # Q6_K gate/up: the per-token routed path, then the shared calls
    (Q4_K, 16, 4, 0, 256, 512, 512, Q4_K),      # no routes: the shared experts alone
    (Q4_K, 16, 4, 3, 256, 512, 0, Q4_K),        # no shared experts: the routed call alone
    (Q4_K, 8, 6, 2, 256, 2304, 512, Q4_K),      # 9 super-blocks: the shared tile's wave 0 takes two
    (Q4_K, 8, 20, 2, 256, 512, 512, Q4_K),      # over 16 tokens: the shared SwiGLU as its own launch
    (Q4_K, 8, 6, 2, 256, 512, 4352, Q4_K),      # 272 shared tiles on 136 workgroups, two each
    (Q4_K, 8, 6, 2, 256, 512, 8448, Q4_K),      # 528 shared tiles, more than two per workgroup: its own launch
])
def test_moe_ffn_matches_three_calls(gu, E, tokens, k, ffn, hid, sffn, stype):
    """The MoE FFN call (routed from the logits, then the shared experts) gives, bit for bit, what the
    routed call from logits followed by qlin_launch_quant_swiglu_rows and qlin_launch_quant_matmul_add
    give on the same inputs, and the per-token reference's routed sum plus the shared experts to 1e-4.
    Up to 16 tokens with Q4_K shared weights, the shared SwiGLU runs inside the routed gate/up launch
    (two 16-row tiles per workgroup from x staged in LDS, the separate kernel's sums in its order); the
    cases over 16 tokens and over two tiles per workgroup take the separate launch."""
    wg, wu, grb, geb, wdn, drb, deb, x, _, _ = _moe_batch(gu, Q5_0, E, ffn, hid, tokens, k, 401 + E + tokens)
    rng = np.random.default_rng(411 + tokens)
    logits = rng.standard_normal((tokens, E)).astype(np.float32)
    if sffn:
        sg, srb, _ = qgen.random_matrix(stype, sffn, hid, seed=421 + sffn)
        su, _, _ = qgen.random_matrix(stype, sffn, hid, seed=422 + sffn)
        sd, sdrb, _ = qgen.random_matrix(stype, hid, sffn, seed=423 + sffn)
    else:
        sg = su = sd = np.zeros(16, np.uint8)
        srb, sdrb = qlin.row_bytes(stype, hid), 0
    out0 = rng.standard_normal((tokens, hid)).astype(np.float32)
    d = {n: dev(v) for n, v in dict(wg=wg, wu=wu, wdn=wdn, x=x, lg=logits, sg=sg, su=su, sd=sd).items()}
    nbytes = qlin.lib().qlin_moe_ffn_workspace_bytes(tokens, k, E, ffn, hid, sffn)
    ws = torch.empty(nbytes + 256, dtype=torch.uint8, device="cuda")
    wsp = (ws.data_ptr() + 255) // 256 * 256
    kk = max(k, 1)
    out_f, ids_f, rw_f = dev(out0), torch.full((tokens, kk), -7, dtype=torch.int32, device="cuda"), empty_f32(tokens, kk)
    banner(f"moe ffn fused gu={gu} E={E} tokens={tokens} k={k} shared={sffn} type {stype}")
    qlin.call("qlin_moe_ffn_decode_grouped_logits", gu, d["wg"], d["wu"], wg.size, Q5_0, d["wdn"], wdn.size, E, ffn,
              hid, hid, stype, d["sg"], d["su"], srb, d["sd"], sdrb, sffn, d["x"], d["lg"], 1.0, ids_f, rw_f, wsp,
              nbytes, out_f, tokens, k)
    out_3, ids_3, rw_3 = dev(out0), torch.full((tokens, kk), -7, dtype=torch.int32, device="cuda"), empty_f32(tokens, kk)
    sact = empty_f32(tokens, max(sffn, 1))
    if k:
        qlin.call("qlin_moe_routed_decode_grouped_logits", gu, d["wg"], d["wu"], wg.size, Q5_0, d["wdn"], wdn.size, E,
                  ffn, hid, hid, d["x"], d["lg"], 1.0, ids_3, rw_3, wsp, nbytes, out_3, tokens, k)
    if sffn:
        qlin.quant_swiglu_rows(stype, d["sg"], d["su"], srb, srb, d["x"], sact, sffn, hid, tokens)
        qlin.quant_matmul_add(stype, d["sd"], sdrb, sact, out_3, hid, sffn, tokens)
    torch.cuda.synchronize()
    assert torch.equal(out_f, out_3)
    if k:
        assert torch.equal(ids_f, ids_3) and torch.equal(rw_f, rw_3)
    ref = out0.copy()
    if k:
        ids_r, _ = orc.router_topk(logits, k, 1.0)
        assert np.array_equal(host(ids_f), ids_r)
        ref = _moe_batch_ref(gu, Q5_0, wg, wu, grb, geb, wdn, drb, deb, x, ids_r, host(rw_f), out0, ffn, hid)
    if sffn:
        for t in range(tokens):
            act = orc.swiglu(stype, sg, su, srb, srb, x[t], sffn, hid).astype(np.float32)
            ref[t] = orc.gemv_add(stype, sd, sdrb, act, ref[t], hid, sffn)
    assert normwise_rel_err(host(out_f) - out0, ref - out0) <= 1e-4


@pytest.mark.parametrize("gu,E,k,ffn,hid,sffn,stype,special", [(*c, None)[:8] for c in [
    (Q4_K, 64, 6, 1408, 2048, 2816, Q4_K),  # DeepSeek-V2-Lite: the shared experts ride in the routed SwiGLU
    (Q4_K, 8, 2, 256, 512, 512, Q4_K),      # same form, two shared blocks
    (Q6_K, 8, 2, 256, 512, 256, Q6_K),      # Q6_K gate/up, one shared block
    (Q4_K, 8, 2, 256, 512, 160, Q8_0),      # shared type differs: the separate calls
    (Q4_K, 8, 2, 512, 512, 768, Q4_K),      # shared_ffn not a multiple of ffn_dim: the separate calls
    (Q4_K, 32, 15, 256, 512, 512, Q4_K),    # 17 routes in all: the separate calls
    (Q4_K, 100, 6, 256, 512, 512, Q4_K),    # over 64 experts: the router launch, then the separate calls
    (Q4_K, 8, 0, 256, 512, 512, Q4_K),      # no routes: the shared experts alone
    (Q4_K, 16, 3, 256, 512, 0, Q4_K),       # no shared experts: the routed call alone
    (Q4_K, 8, 6, 256, 512, 512, Q4_K, "two_finite"),  # 4 empty routes next to the shared blocks
]])
def test_moe_ffn_token_matches_separate_calls(gu, E, k, ffn, hid, sffn, stype, special):
    """The per-token MoE FFN call gives, bit for bit, what the routed call from logits followed by
    qlin_launch_quant_swiglu and qlin_launch_quant_gemv_add on the shared weights give, and the
    oracle's routed sum plus shared experts to 1e-4."""
    wg, grb, geb = _experts(gu, E, ffn, hid, 501 + E)
    wu, _, _ = _experts(gu, E, ffn, hid, 502 + E)
    wdn, drb, deb = _experts(Q5_0, E, hid, ffn, 503 + E)
    rng = np.random.default_rng(504 + k)
    x = rng.standard_normal(hid).astype(np.float32)
    logits = rng.standard_normal((1, E)).astype(np.float32)
    if special == "two_finite":
        logits[0, :] = -np.inf
        logits[0, [E - 1, 2]] = [0.5, 0.25]
    if sffn:
        sg, srb, _ = qgen.random_matrix(stype, sffn, hid, seed=511 + sffn)
        su, _, _ = qgen.random_matrix(stype, sffn, hid, seed=512 + sffn)
        sd, sdrb, _ = qgen.random_matrix(stype, hid, sffn, seed=513 + sffn)
    else:
        sg = su = sd = np.zeros(16, np.uint8)
        srb, sdrb = qlin.row_bytes(stype, hid), 0
    out0 = rng.standard_normal(hid).astype(np.float32)
    d = {n: dev(v) for n, v in dict(wg=wg, wu=wu, wdn=wdn, x=x, lg=logits, sg=sg, su=su, sd=sd).items()}
    kk = max(k, 1)
    out_f, ids_f, rw_f = dev(out0), torch.full((kk,), -7, dtype=torch.int32, device="cuda"), empty_f32(kk)
    act_f = empty_f32(k * ffn + sffn + 1)
    banner(f"moe ffn token gu={gu} E={E} k={k} shared={sffn} type {stype}")
    qlin.call("qlin_moe_ffn_decode_indexed_logits", gu, d["wg"], d["wu"], wg.size, Q5_0, d["wdn"], wdn.size, E, ffn,
              hid, hid, stype, d["sg"], d["su"], srb, d["sd"], sdrb, sffn, d["x"], d["lg"], 0.75, ids_f, rw_f, act_f,
              out_f, k)
    out_s, ids_s, rw_s = dev(out0), torch.full((kk,), -7, dtype=torch.int32, device="cuda"), empty_f32(kk)
    act_s, sact = empty_f32(kk * ffn), empty_f32(max(sffn, 1))
    qlin.call("qlin_moe_routed_decode_indexed_logits", gu, d["wg"], d["wu"], wg.size, Q5_0, d["wdn"], wdn.size, E,
              ffn, hid, hid, d["x"], d["lg"], 0.75, ids_s, rw_s, act_s, out_s, k)
    if sffn:
        qlin.quant_swiglu(stype, d["sg"], d["su"], srb, srb, d["x"], sact, sffn, hid)
        qlin.quant_gemv_add(stype, d["sd"], sdrb, sact, out_s, hid, sffn)
    torch.cuda.synchronize()
    assert torch.equal(out_f, out_s)
    if sffn:
        assert torch.equal(act_f[k * ffn:k * ffn + sffn], sact)
    if k:
        assert torch.equal(ids_f, ids_s) and torch.equal(rw_f, rw_s)
        assert torch.equal(act_f[:k * ffn], act_s[:k * ffn])
    ref = out0.copy()
    if k:
        ids_r, _ = orc.router_topk(logits, k, 0.75)
        assert np.array_equal(host(ids_f), ids_r[0])
        act = orc.swiglu_indexed(gu, wg, wu, geb, geb, grb, grb, x, ids_r[0], ffn, hid)
        ref = orc.down_indexed_ordered(Q5_0, wdn, deb, drb, act, ids_r[0], host(rw_f), out0, hid, ffn)
    if sffn:
        act = orc.swiglu(stype, sg, su, srb, srb, x, sffn, hid).astype(np.float32)
        ref = orc.gemv_add(stype, sd, sdrb, act, ref, hid, sffn)
    assert normwise_rel_err(host(out_f) - out0, ref - out0) <= 1e-4


def test_moe_grouped_wide_input_two_routes_per_pass():
    """in_dim 10240: four routes' staged activations would not fit in LDS, so gate/up runs two routes
    per pass; every expert has more than two routes (4 experts, 8 tokens x 2 routes)."""
    E, ffn, hid, tokens, k = 4, 256, 10240, 8, 2
    wg, wu, grb, geb, wdn, drb, deb, x, ids, rw = _moe_batch(Q4_K, Q5_0, E, ffn, hid, tokens, k, 331)
    out0 = np.zeros((tokens, hid), np.float32)
    banner("moe grouped wide input")
    got = _run_grouped(Q4_K, Q5_0, wg, wu, wdn, E, ffn, hid, x, ids, rw, out0)
    ref = _moe_batch_ref(Q4_K, Q5_0, wg, wu, grb, geb, wdn, drb, deb, x, ids, rw, out0, ffn, hid)
    assert normwise_rel_err(got, ref) <= 1e-4


# ---- batched and fused streaming launches ------------------------------------------------------

def test_gemv_multi_qkv_shapes():
    """q, k, v of a Qwen2-7B layer ([3584|512|512, 3584] Q4_K) in one launch."""
    shapes = [3584, 512, 512]
    mats = [qgen.random_matrix(Q4_K, n, 3584, seed=300 + i) for i, n in enumerate(shapes)]
    x = qgen.random_x(1, 3584, seed=310)
    ys = [empty_f32(n) for n in shapes]
    banner("gemv multi qkv")
    qlin.quant_gemv_multi(Q4_K, [dev(w) for w, _, _ in mats], mats[0][1], dev(x), ys, shapes, 3584)
    for (w, rb, _), y, n in zip(mats, ys, shapes):
        assert normwise_rel_err(host(y), orc.matmul_f64(Q4_K, w, rb, x, n, 3584)[0]) <= FP32


@pytest.mark.parametrize("ffn,hid", [(18944, 3584), (1000, 4608), (7, 256)])
def test_swiglu_stream(ffn, hid):
    wg, rb, _ = qgen.random_matrix(Q4_K, ffn, hid, seed=400 + hid)
    wu, _, _ = qgen.random_matrix(Q4_K, ffn, hid, seed=401 + hid)
    x = qgen.random_x(1, hid, seed=402)[0]
    act_d = empty_f32(ffn)
    banner(f"swiglu stream ffn={ffn} hid={hid}")
    qlin.quant_swiglu(Q4_K, dev(wg), dev(wu), rb, rb, dev(x), act_d, ffn, hid)
    ref = orc.swiglu(Q4_K, wg, wu, rb, rb, x, ffn, hid)
    assert normwise_rel_err(host(act_d), ref) <= 1e-4


@pytest.mark.parametrize("qtype,ffn,hid", [(Q4_0, 18944, 3584), (Q8_0, 4864, 896 + 128), (Q8_0, 4864, 896),
                                          (Q4_0, 9, 256), (Q6_K, 300, 2048), (Q6_K, 17, 768),
                                          (Q6_K, 100, 10240), (Q6_K, 64, 9216 + 256)])
def test_swiglu_matrix_core_formats(qtype, ffn, hid):
    """Fused gate/up SiLU on the 32-weight formats (C2's gate/up pair in one launch) and on Q6_K
    (rows of whole 16-byte units at hid = 2048, of dwords at 768)."""
    sc = 0.02 if qtype == Q4_0 else 0.01  # the Qwen2-7B Q4_0 FFN configuration's block scales
    wg, rb, _ = qgen.random_matrix(qtype, ffn, hid, seed=410 + hid, scale=sc)
    wu, _, _ = qgen.random_matrix(qtype, ffn, hid, seed=411 + hid, scale=sc)
    x = qgen.random_x(1, hid, seed=412)[0]
    act_d = empty_f32(ffn)
    banner(f"swiglu type={qtype} ffn={ffn} hid={hid}")
    qlin.quant_swiglu(qtype, dev(wg), dev(wu), rb, rb, dev(x), act_d, ffn, hid)
    ref = orc.swiglu(qtype, wg, wu, rb, rb, x, ffn, hid)
    assert normwise_rel_err(host(act_d), ref) <= 1e-4


def test_gemv_multi_c3_qkv():
    """C3's q, k, v ([896|128|128, 896] Q8_0, 128-weight chunks) in one matrix-core launch."""
    shapes = [896, 128, 128]
    mats = [qgen.random_matrix(Q8_0, n, 896, seed=520 + i) for i, n in enumerate(shapes)]
    x = qgen.random_x(1, 896, seed=530)
    ys = [empty_f32(n) for n in shapes]
    banner("gemv multi c3 qkv")
    qlin.quant_gemv_multi(Q8_0, [dev(w) for w, _, _ in mats], mats[0][1], dev(x), ys, shapes, 896)
    for (w, rb, _), y, n in zip(mats, ys, shapes):
        assert normwise_rel_err(host(y), orc.matmul_f64(Q8_0, w, rb, x, n, 896)[0]) <= FP32


@pytest.mark.parametrize("qtype,in_dim", [(Q4_K, 256), (Q4_K, 768), (Q4_0, 256), (Q4_0, 512), (Q8_0, 128),
                                          (Q8_0, 384), (Q6_K, 256), (Q6_K, 2048)])
def test_gemv_multi_four_ragged(qtype, in_dim):
    """Four matrices of ragged row counts (1, 17, 33, 300) in one launch: the per-row matrix lookup,
    row slices that end mid-tile, and a single chunk per row at the smallest in_dim."""
    shapes = [17, 1, 33, 300]
    mats = [qgen.random_matrix(qtype, n, in_dim, seed=700 + 13 * i + qtype) for i, n in enumerate(shapes)]
    x = qgen.random_x(1, in_dim, seed=710 + in_dim)
    ys = [empty_f32(n) for n in shapes]
    banner(f"gemv multi four ragged type={qtype} K={in_dim}")
    qlin.quant_gemv_multi(qtype, [dev(w) for w, _, _ in mats], mats[0][1], dev(x), ys, shapes, in_dim)
    for (w, rb, vals), y, n in zip(mats, ys, shapes):
        # a 1-row matrix is a single dot product: judged, as test_gemv_parity does, against its
        # conditioning (sum |w x|) as well as normwise
        yh, ref = host(y), orc.matmul_f64(qtype, w, rb, x, n, in_dim)[0]
        assert normwise_rel_err(yh, ref) <= GATE
        assert cond_err(yh, ref, vals, x) <= COND


def test_gemv_multi_generic_types():
    """Non-Q4_K types take one launch per matrix behind the same entry point."""
    mats = [qgen.random_matrix(Q8_0, n, 512, seed=500 + n) for n in (33, 64)]
    x = qgen.random_x(1, 512, seed=501)
    ys = [empty_f32(33), empty_f32(64)]
    qlin.quant_gemv_multi(Q8_0, [dev(w) for w, _, _ in mats], mats[0][1], dev(x), ys, [33, 64], 512)
    for (w, rb, _), y, n in zip(mats, ys, (33, 64)):
        assert normwise_rel_err(host(y), orc.matmul_f64(Q8_0, w, rb, x, n, 512)[0]) <= FP32


def _pad_rows(w, rows, rb, prb):
    """w's rows (rb bytes each) at a stride of prb bytes, the gap filled with 0xA5."""
    out = np.full((rows, prb), 0xA5, np.uint8)
    out[:, :rb] = w.reshape(rows, rb)
    return out.reshape(-1)


@pytest.mark.gpu
@pytest.mark.parametrize("ffn,extra", [(768, 2), (1024, 4), (1280, 6)])
def test_q6k_padded_rows(ffn, extra):
    """Q6_K rows at a stride past their packed size, a multiple of 4 bytes (so the matrix-core checks
    pass), with an odd or even number of super-blocks per row: the GEMV and the routed down in route
    order (launch_quant_down_f32_indexed_accum_ordered, kernel.cu:1363-1385), every route of every
    parity, against the oracle at the same stride."""
    E, hid = 8, 96
    w, rb, vals = qgen.random_matrix(Q6_K, E * hid, ffn, seed=ffn + 7)
    prb = rb + extra
    assert prb % 4 == 0
    wp = _pad_rows(w, E * hid, rb, prb)
    banner(f"q6k padded rows ffn={ffn} rb={rb} stride={prb}")
    x = qgen.random_x(1, ffn, seed=ffn)
    y = gpu_gemv(Q6_K, wp, prb, x, E * hid, ffn)
    ref = orc.matmul_f64(Q6_K, wp, prb, x, E * hid, ffn)
    assert normwise_rel_err(y, ref) <= GATE
    assert cond_err(y, ref, vals, x) <= COND
    ids = np.array([3, 0, 7, 5, 1, -1, 6], np.int32)
    k = ids.size
    rw = np.linspace(0.3, 0.05, k).astype(np.float32)
    act = np.random.default_rng(ffn).standard_normal((k, ffn)).astype(np.float32)
    out0 = np.random.default_rng(ffn + 1).standard_normal(hid).astype(np.float32)
    out_d = dev(out0)
    qlin.call("qlin_launch_quant_down_f32_indexed_accum_ordered", Q6_K, dev(wp), hid * prb, prb, dev(act), dev(ids),
              dev(rw), out_d, k, hid, ffn)
    ref = orc.down_indexed_ordered(Q6_K, wp, hid * prb, prb, act, ids, rw, out0, hid, ffn)
    got = host(out_d)
    assert normwise_rel_err(got - out0, ref - out0) <= 1e-4
    assert normwise_rel_err(got, ref) <= FP32
