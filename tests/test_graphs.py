"""HIP-graph replays against eager runs: every entry point here is meant to be captured (nothing allocates,
synchronises or reads back), so a captured call is replayed several times, with the program's own eager work
and synchronisations between the replays, and every replay must give the eager result bit for bit (the
kernels sum in fixed orders).  Covers the decode GEMV forms, the fused norm launches, the batched and
per-token MoE calls (workspace, allocation-free and from router logits), the MoE FFN call (routed and shared
experts) and a whole decoder step."""
import numpy as np
import pytest

import oracle as orc
import qgen
from qgen import Q4_K, Q5_0, Q8_0

pytestmark = pytest.mark.gpu

REPLAYS = 3


def _env():
    import torch
    from gpu_util import bind_stream
    assert torch.cuda.is_available(), "GPU tests need the MI355X"
    bind_stream()
    from blog_amd import qlin
    return torch, qlin


def _replays_match(torch, qlin, run, outputs, reset):
    """run() launches the calls on the current stream; outputs() returns the tensors to compare; reset()
    clears them eagerly (it runs between the replays, outside the graph)."""
    reset()
    run()
    torch.cuda.synchronize()
    ref = [o.clone() for o in outputs()]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        qlin.set_stream(torch.cuda.current_stream())
        run()
    qlin.set_stream(torch.cuda.current_stream())
    for i in range(REPLAYS):
        reset()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(outputs(), ref):
            assert torch.equal(a, b), f"replay {i} differs from the eager run"


def test_graph_decode_gemv_forms():
    """The Q4_K decode forms of one layer (q/k/v multi, o add, SwiGLU, down) and a Q8_0 GEMV."""
    torch, qlin = _env()
    from gpu_util import dev, empty_f32
    H, F, KV = 1024, 2816, 256
    mats = {n: qgen.random_matrix(Q4_K, r, c, seed=600 + i)
            for i, (n, r, c) in enumerate([("q", H, H), ("k", KV, H), ("v", KV, H), ("o", H, H), ("g", F, H),
                                           ("u", F, H), ("d", H, F)])}
    w = {n: dev(m[0]) for n, m in mats.items()}
    rb_h, rb_f = mats["q"][1], mats["d"][1]
    w8, rb8, _ = qgen.random_matrix(Q8_0, 512, 1024, seed=610)
    w8d = dev(w8)
    x = dev(qgen.random_x(1, H, seed=611)[0])
    q, k, v, o, act, y, y8 = (empty_f32(n) for n in (H, KV, KV, H, F, H, 512))
    o0 = dev(np.random.default_rng(612).standard_normal(H).astype(np.float32))

    def run():
        qlin.quant_gemv_multi(Q4_K, [w["q"], w["k"], w["v"]], rb_h, x, [q, k, v], [H, KV, KV], H)
        qlin.call("qlin_launch_quant_gemv_add", Q4_K, w["o"], rb_h, q, o, H, H)
        qlin.quant_swiglu(Q4_K, w["g"], w["u"], rb_h, rb_h, x, act, F, H)
        qlin.call("qlin_launch_quant_gemv", Q4_K, w["d"], rb_f, act, y, H, F, 1)
        qlin.call("qlin_launch_quant_gemv", Q8_0, w8d, rb8, x, y8, 512, 1024, 1)

    def reset():
        o.copy_(o0)
        for t in (q, k, v, act, y, y8):
            t.zero_()

    _replays_match(torch, qlin, run, lambda: [q, k, v, o, act, y, y8], reset)


def test_graph_fused_norm_launches():
    torch, qlin = _env()
    from gpu_util import dev, empty_f32
    H, F = 896, 4864
    wq, rb, _ = qgen.random_matrix(Q8_0, 1152, H, seed=620)
    wg, _, _ = qgen.random_matrix(Q8_0, F, H, seed=621)
    wu, _, _ = qgen.random_matrix(Q8_0, F, H, seed=622)
    x = dev((np.random.default_rng(623).standard_normal(H) * 3).astype(np.float32))
    nw = dev((np.random.default_rng(624).standard_normal(H).astype(np.float32).view(np.uint32) >> 16)
             .astype(np.uint16))
    y, act = empty_f32(1152), empty_f32(F)
    wqd, wgd, wud = dev(wq), dev(wg), dev(wu)

    def run():
        qlin.rms_norm_quant_gemv_multi(Q8_0, [wqd], rb, x, nw, 0, 1e-6, 0, [y], [1152], H)
        qlin.call("qlin_launch_rms_norm_quant_swiglu", Q8_0, wgd, wud, rb, x, nw, 0, 1e-6, 0, act, F, H)

    def reset():
        y.zero_()
        act.zero_()

    _replays_match(torch, qlin, run, lambda: [y, act], reset)


def _moe_mats(E, ffn, hid, seed):
    wg, grb, _ = qgen.random_matrix(Q4_K, E * ffn, hid, seed=seed)
    wu, _, _ = qgen.random_matrix(Q4_K, E * ffn, hid, seed=seed + 1)
    wd, drb, _ = qgen.random_matrix(Q5_0, E * hid, ffn, seed=seed + 2)
    return wg, wu, wd


@pytest.mark.parametrize("form", ["workspace", "noalloc", "logits"])
def test_graph_moe_grouped(form):
    """The batched MoE decode (its gate/up launch groups the routes itself; from logits it also routes)."""
    torch, qlin = _env()
    from gpu_util import dev, empty_f32
    E, ffn, hid, tokens, k = 16, 256, 512, 8, 4
    wg, wu, wd = _moe_mats(E, ffn, hid, 630)
    wgd, wud, wdd = dev(wg), dev(wu), dev(wd)
    rng = np.random.default_rng(633)
    x = dev(rng.standard_normal((tokens, hid)).astype(np.float32))
    logits_h = rng.standard_normal((tokens, E)).astype(np.float32)
    ids_h, rw_h = orc.router_topk(logits_h, k, 1.0)
    logits, ids, rw = dev(logits_h), dev(ids_h), dev(rw_h)
    out0 = dev(rng.standard_normal((tokens, hid)).astype(np.float32))
    out = empty_f32(tokens, hid)
    ids_o = torch.zeros((tokens, k), dtype=torch.int32, device="cuda")
    rw_o = empty_f32(tokens, k)
    nbytes = qlin.lib().qlin_moe_grouped_workspace_bytes(tokens, k, E, ffn, hid)
    ws = torch.empty(nbytes + 256, dtype=torch.uint8, device="cuda")
    wsp = (ws.data_ptr() + 255) // 256 * 256

    def run():
        if form == "workspace":
            qlin.call("qlin_moe_routed_decode_grouped", Q4_K, wgd, wud, wg.size, Q5_0, wdd, wd.size, E, ffn, hid, hid,
                      x, ids, rw, wsp, nbytes, out, tokens, k)
        elif form == "noalloc":
            qlin.call("qlin_moe_routed_decode_grouped_noalloc", Q4_K, wgd, wud, wg.size, Q5_0, wdd, wd.size, E, ffn,
                      hid, hid, x, ids, rw, out, tokens, k)
        else:
            qlin.call("qlin_moe_routed_decode_grouped_logits", Q4_K, wgd, wud, wg.size, Q5_0, wdd, wd.size, E, ffn,
                      hid, hid, x, logits, 1.0, ids_o, rw_o, wsp, nbytes, out, tokens, k)

    def reset():
        out.copy_(out0)
        ids_o.fill_(-3)
        rw_o.zero_()

    _replays_match(torch, qlin, run, lambda: [out, ids_o, rw_o], reset)


def test_graph_moe_ffn():
    """The MoE FFN call (routed from the logits, shared experts, the routed sum added in the shared down-add)."""
    torch, qlin = _env()
    from gpu_util import dev, empty_f32
    E, ffn, hid, tokens, k, sffn = 16, 256, 512, 8, 4, 512
    wg, wu, wd = _moe_mats(E, ffn, hid, 650)
    sg, srb, _ = qgen.random_matrix(Q4_K, sffn, hid, seed=654)
    su, _, _ = qgen.random_matrix(Q4_K, sffn, hid, seed=655)
    sd, sdrb, _ = qgen.random_matrix(Q4_K, hid, sffn, seed=656)
    wgd, wud, wdd, sgd, sud, sdd = (dev(a) for a in (wg, wu, wd, sg, su, sd))
    rng = np.random.default_rng(657)
    x = dev(rng.standard_normal((tokens, hid)).astype(np.float32))
    logits = dev(rng.standard_normal((tokens, E)).astype(np.float32))
    out0 = dev(rng.standard_normal((tokens, hid)).astype(np.float32))
    out = empty_f32(tokens, hid)
    ids_o = torch.zeros((tokens, k), dtype=torch.int32, device="cuda")
    rw_o = empty_f32(tokens, k)
    nbytes = qlin.lib().qlin_moe_ffn_workspace_bytes(tokens, k, E, ffn, hid, sffn)
    ws = torch.empty(nbytes + 256, dtype=torch.uint8, device="cuda")
    wsp = (ws.data_ptr() + 255) // 256 * 256

    def run():
        qlin.call("qlin_moe_ffn_decode_grouped_logits", Q4_K, wgd, wud, wg.size, Q5_0, wdd, wd.size, E, ffn, hid, hid,
                  Q4_K, sgd, sud, srb, sdd, sdrb, sffn, x, logits, 1.0, ids_o, rw_o, wsp, nbytes, out, tokens, k)

    def reset():
        out.copy_(out0)
        ids_o.fill_(-3)
        rw_o.zero_()

    _replays_match(torch, qlin, run, lambda: [out, ids_o, rw_o], reset)


def test_graph_moe_token_from_logits():
    torch, qlin = _env()
    from gpu_util import dev, empty_f32
    E, ffn, hid, k = 32, 256, 512, 6
    wg, wu, wd = _moe_mats(E, ffn, hid, 640)
    wgd, wud, wdd = dev(wg), dev(wu), dev(wd)
    rng = np.random.default_rng(643)
    x = dev(rng.standard_normal(hid).astype(np.float32))
    logits = dev(rng.standard_normal(E).astype(np.float32))
    out0 = dev(rng.standard_normal(hid).astype(np.float32))
    out, act, rw = empty_f32(hid), empty_f32(k, ffn), empty_f32(k)
    ids = torch.zeros(k, dtype=torch.int32, device="cuda")

    def run():
        qlin.call("qlin_moe_routed_decode_indexed_logits", Q4_K, wgd, wud, wg.size, Q5_0, wdd, wd.size, E, ffn, hid,
                  hid, x, logits, 1.0, ids, rw, act, out, k)

    def reset():
        out.copy_(out0)
        ids.fill_(-3)
        rw.zero_()
        act.zero_()

    _replays_match(torch, qlin, run, lambda: [out, ids, rw, act], reset)


def test_graph_moe_ffn_token():
    """The per-token MoE FFN call with the shared experts in the routed SwiGLU launch."""
    torch, qlin = _env()
    from gpu_util import dev, empty_f32
    E, ffn, hid, k, sffn = 32, 256, 512, 6, 512
    wg, wu, wd = _moe_mats(E, ffn, hid, 660)
    sg, srb, _ = qgen.random_matrix(Q4_K, sffn, hid, seed=664)
    su, _, _ = qgen.random_matrix(Q4_K, sffn, hid, seed=665)
    sd, sdrb, _ = qgen.random_matrix(Q4_K, hid, sffn, seed=666)
    wgd, wud, wdd, sgd, sud, sdd = (dev(a) for a in (wg, wu, wd, sg, su, sd))
    rng = np.random.default_rng(667)
    x = dev(rng.standard_normal(hid).astype(np.float32))
    logits = dev(rng.standard_normal(E).astype(np.float32))
    out0 = dev(rng.standard_normal(hid).astype(np.float32))
    out, act, rw = empty_f32(hid), empty_f32(k * ffn + sffn), empty_f32(k)
    ids = torch.zeros(k, dtype=torch.int32, device="cuda")

    def run():
        qlin.call("qlin_moe_ffn_decode_indexed_logits", Q4_K, wgd, wud, wg.size, Q5_0, wdd, wd.size, E, ffn, hid, hid,
                  Q4_K, sgd, sud, srb, sdd, sdrb, sffn, x, logits, 1.0, ids, rw, act, out, k)

    def reset():
        out.copy_(out0)
        ids.fill_(-3)
        rw.zero_()
        act.zero_()

    _replays_match(torch, qlin, run, lambda: [out, ids, rw, act], reset)


def test_graph_decoder_steps_match_eager():
    """A small Qwen2-architecture decoder (fused norms and rotary): the step captured once and replayed
    gives, step after step, the eager decoder's logits and tokens (the step reads its token and position
    from device memory and advances them)."""
    torch, qlin = _env()
    from blog_amd.decoder import Qwen2Config, Qwen2Decoder, make_weights
    cfg = Qwen2Config(layers=2, vocab=4096)
    w = make_weights(torch, cfg, seed=77)
    prompt = torch.randint(0, cfg.vocab, (6,), dtype=torch.int32, device="cuda",
                           generator=torch.Generator(device="cuda").manual_seed(5))
    n = 5
    eager = Qwen2Decoder(torch, cfg, w, max_seq=32, max_prompt=8)
    ref_logits = torch.zeros(n, cfg.vocab, device="cuda")
    ref_toks = eager.generate(prompt, n, logits_out=ref_logits)
    dec = Qwen2Decoder(torch, cfg, w, max_seq=32, max_prompt=8)
    dec.prefill(prompt)
    torch.cuda.synchronize()
    assert torch.equal(dec.logits, ref_logits[0])
    # capture without running: the graph's first replay is the first step
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        dec.step()
    qlin.set_stream(torch.cuda.current_stream())
    toks = [int(dec.token.item())]
    for i in range(1, n):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(dec.logits, ref_logits[i]), f"step {i}"
        toks.append(int(dec.token.item()))
    assert toks == ref_toks
