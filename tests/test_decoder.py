"""Benchmark configuration C3: a Qwen2.5-0.5B-architecture decoder with every linear in Q8_0, greedy decoding.

CPU: the oracle's decoder twin (orc_qwen2_logits) pinned by an independent numpy restatement of the
layer on a small model (every index: GQA head mapping, rotary pairs, causal window, tied head), and
by closed forms (one position attends to itself only, so the query and key weights cannot matter).
GPU: the glue kernels (include/qlin_decoder.h) against numpy, and the whole decoder
(blog_amd/decoder.py) on its 32-token prompt plus 128 greedy tokens, teacher-forced against the twin:
every step's logits within 1e-3 normwise, and the greedy tokens counted against the twin's picks.
"""
import numpy as np
import pytest

import oracle as orc
import qgen
from qgen import Q8_0, normwise_rel_err

SMALL = dict(layers=2, hidden=64, n_heads=4, kv_heads=2, head_dim=16, ffn=96, vocab=40, wtype=Q8_0,
             eps=1e-6, theta=10000.0)


def _small_model(cfg, seed):
    rng = np.random.default_rng(seed)
    H, F, QD, KD = cfg["hidden"], cfg["ffn"], cfg["n_heads"] * cfg["head_dim"], cfg["kv_heads"] * cfg["head_dim"]

    def lin(n, k):
        w, _, vals = qgen.random_matrix(Q8_0, n, k, seed=int(rng.integers(1 << 30)), scale=0.05)
        return w, vals.astype(np.float64)

    layers, vals = [], []
    for _ in range(cfg["layers"]):
        L, V = {}, {}
        for name, n, k in (("wq", QD, H), ("wk", KD, H), ("wv", KD, H), ("wo", H, QD), ("wg", F, H), ("wu", F, H),
                           ("wd", H, F)):
            L[name], V[name] = lin(n, k)
        L["attn_norm"] = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
        L["ffn_norm"] = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
        layers.append(L)
        vals.append(V)
    table, tvals = lin(cfg["vocab"], H)
    final = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    return layers, vals, final, table, tvals


def _numpy_decoder(cfg, layers, vals, final, tvals, tokens, first):
    """The Qwen2 layer written out in numpy float64 from the published architecture."""
    H, NH, NKV, D = cfg["hidden"], cfg["n_heads"], cfg["kv_heads"], cfg["head_dim"]
    eps, theta = cfg["eps"], cfg["theta"]

    def norm(x, w):
        return x / np.sqrt(np.mean(x * x) + eps) * w.astype(np.float64)

    def rope(x, pos):  # x [heads, D]
        half = D // 2
        ang = pos / theta ** (np.arange(half) * 2.0 / D)
        c, s = np.cos(ang), np.sin(ang)
        a, b = x[:, :half].copy(), x[:, half:].copy()
        return np.concatenate([a * c - b * s, b * c + a * s], axis=1)

    ks = [[] for _ in layers]
    vs = [[] for _ in layers]
    out = []
    for pos, tok in enumerate(tokens):
        h = tvals[tok].copy()
        for li, V in enumerate(vals):
            L = layers[li]
            xn = norm(h, L["attn_norm"])
            q = rope((V["wq"] @ xn).reshape(NH, D), pos)
            k = rope((V["wk"] @ xn).reshape(NKV, D), pos)
            ks[li].append(k)
            vs[li].append((V["wv"] @ xn).reshape(NKV, D))
            K, Vv = np.stack(ks[li]), np.stack(vs[li])  # [pos + 1, NKV, D]
            att = np.empty((NH, D))
            for hh in range(NH):
                kh = hh // (NH // NKV)
                sc = K[:, kh, :] @ q[hh] / np.sqrt(D)
                p = np.exp(sc - sc.max())
                att[hh] = (p / p.sum()) @ Vv[:, kh, :]
            h = h + V["wo"] @ att.reshape(-1)
            xn = norm(h, L["ffn_norm"])
            g, u = V["wg"] @ xn, V["wu"] @ xn
            h = h + V["wd"] @ (g / (1 + np.exp(-g)) * u)
        if pos >= first:
            out.append(tvals @ norm(h, final))
    return np.array(out)


def test_twin_against_numpy_restatement():
    cfg = SMALL
    layers, vals, final, table, tvals = _small_model(cfg, 3)
    tokens = [5, 17, 0, 39, 5, 22, 8]
    got = orc.qwen2_logits(cfg, layers, final, table, tokens, first=2, threads=2)
    ref = _numpy_decoder(cfg, layers, vals, final, tvals, tokens, first=2)
    assert got.shape == (5, cfg["vocab"])
    assert normwise_rel_err(got, ref) <= 1e-6


def test_twin_first_position_ignores_query_and_key():
    """Position 0 attends to itself alone (softmax of one score is 1), so its logits cannot depend on
    the query and key weights; position 1's do."""
    cfg = SMALL
    layers, _, final, table, _ = _small_model(cfg, 4)
    other = [dict(L) for L in layers]
    for L in other:
        L["wq"] = qgen.random_matrix(Q8_0, cfg["n_heads"] * cfg["head_dim"], cfg["hidden"], seed=99)[0]
        L["wk"] = qgen.random_matrix(Q8_0, cfg["kv_heads"] * cfg["head_dim"], cfg["hidden"], seed=98)[0]
    a = orc.qwen2_logits(cfg, layers, final, table, [7, 3], first=0, threads=1)
    b = orc.qwen2_logits(cfg, other, final, table, [7, 3], first=0, threads=1)
    assert np.array_equal(a[0], b[0])
    assert not np.allclose(a[1], b[1])


# ---- GPU ----------------------------------------------------------------------------------------

def _gpu():
    import torch
    from gpu_util import bind_stream
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    bind_stream()
    return torch


@pytest.mark.gpu
@pytest.mark.parametrize("rows,hidden,wtype,one_plus", [(1, 896, 0, 0), (32, 896, 0, 0), (3, 5000, 1, 1)])
def test_rms_norm(rows, hidden, wtype, one_plus):
    torch = _gpu()
    from gpu_util import banner, dev, empty_f32, host
    from blog_amd import qlin
    rng = np.random.default_rng(hidden + rows)
    x = rng.standard_normal((rows, hidden)).astype(np.float32) * 3
    w16 = (rng.standard_normal(hidden) * 0.5 + 1).astype(np.float16)
    if wtype == 0:
        bits = (w16.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        wv = (bits.astype(np.uint32) << 16).view(np.float32)
    else:
        bits, wv = w16.view(np.uint16), w16.astype(np.float32)
    banner(f"rms_norm rows={rows} hidden={hidden}")
    out = empty_f32(rows, hidden)
    qlin.call("qlin_launch_rms_norm", dev(x), out, dev(bits), wtype, rows, hidden, 1e-6, one_plus)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt(np.mean(x64 * x64, axis=1, keepdims=True) + 1e-6) * (wv.astype(np.float64) + one_plus)
    assert normwise_rel_err(host(out), ref) <= 1e-6


@pytest.mark.gpu
@pytest.mark.parametrize("start,D", [(0, 64), (37, 64), (300, 64), (600, 64), (5, 128), (200, 256)])
def test_rope_attend_one_row(start, D):
    """The decode row's rotary embedding, cache store and attention in one launch: the same caches and
    the same output, bit for bit, as qlin_launch_rope_store_kv followed by qlin_launch_attend (a
    position past the cache clamped to its last slot); q itself is left unrotated."""
    torch = _gpu()
    from gpu_util import banner, dev, empty_f32, host
    from blog_amd import qlin
    NH, NKV, S, theta = 14, 2, 512, 1e6
    rng = np.random.default_rng(start * 7 + D)
    q = rng.standard_normal((1, NH * D)).astype(np.float32)
    k = rng.standard_normal((1, NKV * D)).astype(np.float32)
    v = rng.standard_normal((1, NKV * D)).astype(np.float32)
    kc0 = rng.standard_normal((S, NKV * D)).astype(np.float32)
    vc0 = rng.standard_normal((S, NKV * D)).astype(np.float32)
    pos = torch.tensor([start], dtype=torch.int32, device="cuda")
    banner(f"rope_attend start={start} D={D}")
    qa, kca, vca, attn_a = dev(q), dev(kc0), dev(vc0), empty_f32(1, NH * D)
    qlin.call("qlin_launch_rope_store_kv", qa, dev(k), dev(v), kca, vca, 1, NH, NKV, D, S, pos, theta)
    qlin.call("qlin_launch_attend", qa, kca, vca, attn_a, 1, NH, NKV, D, S, pos)
    qb, kcb, vcb, attn_b = dev(q), dev(kc0), dev(vc0), empty_f32(1, NH * D)
    qlin.call("qlin_launch_rope_attend", qb, dev(k), dev(v), kcb, vcb, attn_b, NH, NKV, D, S, pos, theta)
    assert np.array_equal(host(attn_b), host(attn_a))
    assert np.array_equal(host(kcb), host(kca))
    assert np.array_equal(host(vcb), host(vca))
    assert np.array_equal(host(qb), q)


@pytest.mark.gpu
def test_c3_decode_fused_matches_unfused():
    """The decode step with its norms inside the linears and the rotary embedding inside the attention
    gives the two-launch decoder's logits and tokens."""
    torch = _gpu()
    from gpu_util import banner
    from blog_amd.decoder import Qwen2Config, Qwen2Decoder, make_weights
    cfg = Qwen2Config()
    w = make_weights(torch, cfg, seed=11)
    prompt = torch.randint(0, cfg.vocab, (8,), dtype=torch.int32, device="cuda",
                           generator=torch.Generator(device="cuda").manual_seed(3))
    out = []
    for fuse in (True, False):
        banner(f"c3 decoder fuse={fuse}")
        dec = Qwen2Decoder(torch, cfg, w, max_seq=64, max_prompt=8, fuse=fuse)
        logits = torch.zeros(16, cfg.vocab, device="cuda")
        toks = dec.generate(prompt, 16, logits_out=logits)
        out.append((toks, logits.cpu().numpy()))
    assert out[0][0] == out[1][0]
    assert max(normwise_rel_err(a, b) for a, b in zip(out[0][1], out[1][1])) <= 1e-5


def _norm_weights(rng, hidden, wtype):
    w16 = (rng.standard_normal(hidden) * 0.5 + 1).astype(np.float16)
    if wtype == 0:
        bits = (w16.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
        return bits, (bits.astype(np.uint32) << 16).view(np.float32)
    return w16.view(np.uint16), w16.astype(np.float32)


def _rms_ref(x, wv, one_plus):
    x64 = x.astype(np.float64)
    return (x64 / np.sqrt(np.mean(x64 * x64) + 1e-6) * (wv.astype(np.float64) + one_plus)).astype(np.float32)


@pytest.mark.gpu
@pytest.mark.parametrize("qtype,hidden,outs,wtype,one_plus", [
    (qgen.Q8_0, 896, [896, 128, 128], 0, 0),      # C3's q/k/v
    (qgen.Q8_0, 896, [151936], 0, 0),             # C3's tied head
    (qgen.Q4_K, 3584, [3584, 512, 512], 1, 1),
    (qgen.Q6_K, 1024, [300], 0, 1),
    (qgen.Q5_0, 1152, [200], 1, 0),
    (qgen.Q4_0, 768, [40, 88], 0, 0)])
def test_rms_norm_fused_gemv(qtype, hidden, outs, wtype, one_plus):
    """The RMSNorm inside the decode GEMV's staging: y = W rms_norm(x), against the oracle's product
    with the normalized x, and against the two launches it replaces."""
    torch = _gpu()
    from gpu_util import banner, dev, empty_f32, host
    from blog_amd import qlin
    rng = np.random.default_rng(hidden + len(outs))
    x = (rng.standard_normal(hidden) * 3).astype(np.float32)
    bits, wv = _norm_weights(rng, hidden, wtype)
    mats = [qgen.random_matrix(qtype, n, hidden, seed=500 + i) for i, n in enumerate(outs)]
    rb = mats[0][1]
    ys = [empty_f32(n) for n in outs]
    banner(f"rms_norm fused gemv type={qtype} hidden={hidden} outs={outs}")
    qlin.rms_norm_quant_gemv_multi(qtype, [dev(w) for w, _, _ in mats], rb, dev(x), dev(bits), wtype, 1e-6,
                                   one_plus, ys, outs, hidden)
    xn = _rms_ref(x, wv, one_plus)
    xn_d, ys2 = empty_f32(1, hidden), [empty_f32(n) for n in outs]
    qlin.call("qlin_launch_rms_norm", dev(x), xn_d, dev(bits), wtype, 1, hidden, 1e-6, one_plus)
    qlin.quant_gemv_multi(qtype, [dev(w) for w, _, _ in mats], rb, xn_d, ys2, outs, hidden)
    for (w, _, _), y, y2, n in zip(mats, ys, ys2, outs):
        ref = orc.matmul_f64(qtype, w, rb, xn[None, :], n, hidden)[0]
        assert normwise_rel_err(host(y), ref) <= 1e-5
        assert normwise_rel_err(host(y), host(y2)) <= 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("qtype,hidden,vocab,norm,case", [
    (qgen.Q8_0, 896, 151936, True, "random"),   # C3's tied head with the final norm
    (qgen.Q8_0, 896, 151936, True, "tie"),      # the largest logit twice: the lower row wins
    (qgen.Q4_K, 1024, 3000, False, "random"),
    (qgen.Q6_K, 1024, 4100, False, "tie"),
    (qgen.Q5_0, 1152, 777, True, "random"),
    (qgen.Q8_0, 896, 5000, False, "nan"),       # every third row's logit NaN (a NaN block scale): never picked
    (qgen.Q8_0, 896, 300, False, "allnan"),     # every logit NaN: nothing beats -inf, index 0
    (qgen.Q4_K, 1024, 8704, False, "tail_tie"),  # 2 whole tiles and 2 rows per workgroup: the largest logit
                                                 # in two workgroups' last rows, the lower row wins
])
def test_gemv_argmax(qtype, hidden, vocab, norm, case):
    """The head GEMV with the greedy pick in its epilogue: the logits are the plain launches' bit for bit,
    and the index is qlin_launch_argmax's over them (and numpy's first maximum when nothing is NaN)."""
    torch = _gpu()
    from gpu_util import banner, dev, empty_f32, host
    from blog_amd import qlin
    rng = np.random.default_rng(vocab + hidden)
    x = (rng.standard_normal(hidden) * 3).astype(np.float32)
    bits, _ = _norm_weights(rng, hidden, 0)
    w, rb, _ = qgen.random_matrix(qtype, vocab, hidden, seed=530 + vocab)
    if case in ("nan", "allnan"):
        # Q8_0 block 0 of the chosen rows gets the f16 NaN 0x7e00 as its scale
        w = w.copy()
        rows = w.reshape(vocab, rb)
        chosen = rows if case == "allnan" else rows[1::3]
        chosen[:, 0:2] = [0x00, 0x7e]
    if case == "tail_tie":
        # the largest logit's row copied into rows 8195 and 8492, past the whole tiles (in the last rows
        # of workgroups 1 and 150 when every workgroup takes 2 whole tiles and then 2 rows)
        lg = empty_f32(vocab)
        qlin.call("qlin_launch_quant_gemv", qtype, dev(w), rb, dev(x), lg, vocab, hidden, 1)
        top = int(np.argmax(host(lg)))
        w = w.copy()
        rows = w.reshape(vocab, rb)
        src = rows[top].copy()
        if top not in (8195, 8492):
            rows[top] = rows[0 if top else 1]  # the maximum now only in the two copies
        rows[8195] = src
        rows[8492] = src
    if case == "tie":
        # copy the row of the largest logit into a row below it: two equal logits
        lg = empty_f32(vocab)
        if norm:
            qlin.rms_norm_quant_gemv_multi(qtype, [dev(w)], rb, dev(x), dev(bits), 0, 1e-6, 0, [lg], [vocab], hidden)
        else:
            qlin.call("qlin_launch_quant_gemv", qtype, dev(w), rb, dev(x), lg, vocab, hidden, 1)
        top = int(np.argmax(host(lg)))
        low = top // 2 if top > 0 else 1
        w = w.copy()
        w.reshape(vocab, rb)[min(low, top)] = w.reshape(vocab, rb)[max(low, top)]
    wd, xd, nd = dev(w), dev(x), dev(bits) if norm else None
    logits, idx = empty_f32(vocab), torch.full((1,), -5, dtype=torch.int32, device="cuda")
    scratch = torch.empty(8192, dtype=torch.uint8, device="cuda")
    banner(f"gemv argmax type={qtype} hidden={hidden} vocab={vocab} norm={norm} case={case}")
    qlin.call("qlin_launch_quant_gemv_argmax", qtype, wd, rb, xd, nd if norm else 0, 0, 1e-6, 0, logits, vocab, hidden,
              scratch, idx)
    ref_lg, ref_idx = empty_f32(vocab), torch.full((1,), -5, dtype=torch.int32, device="cuda")
    if norm:
        qlin.rms_norm_quant_gemv_multi(qtype, [wd], rb, xd, nd, 0, 1e-6, 0, [ref_lg], [vocab], hidden)
    else:
        qlin.call("qlin_launch_quant_gemv", qtype, wd, rb, xd, ref_lg, vocab, hidden, 1)
    qlin.call("qlin_launch_argmax", ref_lg, vocab, ref_idx)
    torch.cuda.synchronize()
    assert torch.equal(logits.view(torch.int32), ref_lg.view(torch.int32))  # bit for bit, NaNs included
    got = int(host(idx)[0])
    assert got == int(host(ref_idx)[0])
    h = host(logits)
    if case == "allnan":
        assert np.isnan(h).all() and got == 0
    elif case == "nan":
        assert np.isnan(h[1::3]).all() and not np.isnan(h[0::3]).any()
        assert got == int(np.nanargmax(h))
    else:
        assert got == int(np.argmax(h))
    if case == "tie":
        assert (h == h[got]).sum() >= 2 and got == int(np.flatnonzero(h == h.max())[0])
    if case == "tail_tie":
        assert h[8195] == h[8492] == h.max() and got == 8195


@pytest.mark.gpu
@pytest.mark.parametrize("qtype,hidden,ffn", [(qgen.Q8_0, 896, 4864), (qgen.Q4_K, 3584, 18944), (qgen.Q4_0, 512, 100)])
def test_rms_norm_fused_swiglu(qtype, hidden, ffn):
    torch = _gpu()
    from gpu_util import banner, dev, empty_f32, host
    from blog_amd import qlin
    rng = np.random.default_rng(hidden + ffn)
    x = (rng.standard_normal(hidden) * 3).astype(np.float32)
    bits, wv = _norm_weights(rng, hidden, 0)
    wg, rb, _ = qgen.random_matrix(qtype, ffn, hidden, seed=520)
    wu, _, _ = qgen.random_matrix(qtype, ffn, hidden, seed=521)
    act = empty_f32(ffn)
    banner(f"rms_norm fused swiglu type={qtype} hidden={hidden} ffn={ffn}")
    qlin.call("qlin_launch_rms_norm_quant_swiglu", qtype, dev(wg), dev(wu), rb, dev(x), dev(bits), 0, 1e-6, 0, act,
              ffn, hidden)
    ref = orc.swiglu(qtype, wg, wu, rb, rb, _rms_ref(x, wv, 0), ffn, hidden)
    assert normwise_rel_err(host(act), ref) <= 1e-4


@pytest.mark.gpu
def test_rms_norm_fused_unsupported_shape():
    """An in_dim the matrix-core decode kernels do not take is refused, not run."""
    torch = _gpu()
    from gpu_util import dev, empty_f32
    from blog_amd import qlin
    w, rb, _ = qgen.random_matrix(qgen.Q8_0, 16, 96, seed=530)
    x = np.ones(96, np.float32)
    bits = np.full(96, 0x3f80, np.uint16)
    y = empty_f32(16)
    rc = qlin.status("qlin_launch_rms_norm_quant_swiglu", qgen.Q8_0, dev(w), dev(w), rb, dev(x), dev(bits), 0, 1e-6,
                     0, y, 16, 96)
    assert rc == 5  # QLIN_ERR_LIMIT


@pytest.mark.gpu
@pytest.mark.parametrize("rows,start", [(1, 0), (1, 37), (32, 0), (5, 250), (3, 509), (1, 600)])
def test_rope_store_and_attend(rows, start):
    """Rotary pairs, the cache store at each row's position (a position past the cache clamped to its
    last slot), and causal GQA attention (14 query heads over 2 KV heads of 64) against numpy float64."""
    torch = _gpu()
    from gpu_util import banner, dev, empty_f32, host
    from blog_amd import qlin
    NH, NKV, D, S, theta = 14, 2, 64, 512, 1e6
    rng = np.random.default_rng(rows * 1000 + start)
    q = rng.standard_normal((rows, NH * D)).astype(np.float32)
    k = rng.standard_normal((rows, NKV * D)).astype(np.float32)
    v = rng.standard_normal((rows, NKV * D)).astype(np.float32)
    kc0 = rng.standard_normal((S, NKV * D)).astype(np.float32)  # earlier positions' keys and values
    vc0 = rng.standard_normal((S, NKV * D)).astype(np.float32)
    banner(f"rope/attend rows={rows} start={start}")
    qd, kcd, vcd = dev(q), dev(kc0), dev(vc0)
    pos = torch.tensor([start], dtype=torch.int32, device="cuda")
    qlin.call("qlin_launch_rope_store_kv", qd, dev(k), dev(v), kcd, vcd, rows, NH, NKV, D, S, pos, theta)
    attn = empty_f32(rows, NH * D)
    qlin.call("qlin_launch_attend", qd, kcd, vcd, attn, rows, NH, NKV, D, S, pos)

    def rope(x, p):
        half = D // 2
        ang = p / theta ** (np.arange(half) * 2.0 / D)
        c, s = np.cos(ang), np.sin(ang)
        x = x.reshape(-1, D).astype(np.float64)
        return np.concatenate([x[:, :half] * c - x[:, half:] * s, x[:, half:] * c + x[:, :half] * s], axis=1)

    kc, vc = kc0.astype(np.float64).copy(), vc0.astype(np.float64).copy()
    qr = np.empty((rows, NH, D))
    for r in range(rows):
        p = min(start + r, S - 1)
        qr[r] = rope(q[r], p)
        kc[p] = rope(k[r], p).reshape(-1)
        vc[p] = v[r]
    assert normwise_rel_err(host(qd).reshape(rows, NH, D), qr) <= 1e-5
    assert normwise_rel_err(host(kcd), kc) <= 1e-5
    assert np.array_equal(host(vcd), vc.astype(np.float32))
    ref = np.empty((rows, NH, D))
    for r in range(rows):
        p = min(start + r, S - 1)
        for h in range(NH):
            kh = h // (NH // NKV)
            sc = kc[:p + 1].reshape(p + 1, NKV, D)[:, kh] @ qr[r, h] / np.sqrt(D)
            w = np.exp(sc - sc.max())
            ref[r, h] = (w / w.sum()) @ vc[:p + 1].reshape(p + 1, NKV, D)[:, kh]
    assert normwise_rel_err(host(attn).reshape(rows, NH, D), ref) <= 1e-5


@pytest.mark.gpu
def test_c3_greedy_decode_teacher_forced():
    """Config 3 end to end: random Qwen2.5-0.5B-architecture weights in Q8_0, a 32-token uniform
    prompt, 128 greedy tokens.  The twin, fed the same tokens, gives every step's logits within 1e-3
    normwise; its greedy picks are counted against the GPU's."""
    torch = _gpu()
    from gpu_util import banner
    from blog_amd.decoder import Qwen2Config, Qwen2Decoder, make_weights
    cfg = Qwen2Config()
    banner("c3 decoder: weights")
    w = make_weights(torch, cfg, seed=2024)
    dec = Qwen2Decoder(torch, cfg, w, max_seq=256, max_prompt=32)
    prompt = torch.randint(0, cfg.vocab, (32,), dtype=torch.int32, device="cuda",
                           generator=torch.Generator(device="cuda").manual_seed(7))
    n_new = 128
    logits = torch.zeros(n_new, cfg.vocab, device="cuda")
    banner("c3 decoder: prefill + 128 greedy steps")
    toks = dec.generate(prompt, n_new, logits_out=logits)
    torch.cuda.synchronize()
    banner("c3 decoder: twin, teacher-forced")

    def h(t):
        return t.cpu().numpy()

    def bf16_values(t):
        return (h(t).view(np.uint16).astype(np.uint32) << 16).view(np.float32)

    layers = [{n: h(L[n]) for n in ("wq", "wk", "wv", "wo", "wg", "wu", "wd")} |
              {"attn_norm": bf16_values(L["attn_norm"]), "ffn_norm": bf16_values(L["ffn_norm"])}
              for L in w["layers"]]
    c = dict(layers=cfg.layers, hidden=cfg.hidden, n_heads=cfg.n_heads, kv_heads=cfg.kv_heads,
             head_dim=cfg.head_dim, ffn=cfg.ffn, vocab=cfg.vocab, wtype=cfg.wtype, eps=cfg.eps, theta=cfg.theta)
    seq = h(prompt).tolist() + toks[:-1]
    ref = orc.qwen2_logits(c, layers, bf16_values(w["final_norm"]), h(w["table"]), seq, first=31)
    got = h(logits)
    errs = [normwise_rel_err(got[i], ref[i]) for i in range(n_new)]
    matches = sum(int(np.argmax(ref[i]) == toks[i]) for i in range(n_new))
    print(f"[c3] max per-step normwise logits error {max(errs):.2e}; greedy tokens matching the twin: "
          f"{matches}/{n_new}", flush=True)
    assert max(errs) <= 1e-3
    assert matches >= n_new - 2
