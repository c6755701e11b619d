"""A Qwen2-architecture decoder over the quantized-linear path: the harness of benchmark configuration C3.

Qwen2.5-0.5B architecture (24 layers, hidden 896, 14 query / 2 KV heads of 64, SwiGLU FFN 4864,
vocabulary 151936, RMSNorm eps 1e-6, rotary theta 1e6), every linear in Q8_0, random-init weights
N(0, 0.02) before quantization (ggml's Q8_0 rule: d = amax / 127 stored as f16, q = round(x / d), ties
away from zero).  The embedding table is tied to the output head and quantized like the linears, so
the lookup dequantizes one Q8_0 row (qlin_launch_quant_embedding) and the head is a Q8_0 GEMV.  No
q/k/v biases.  Norm weights are bf16 values 1 + N(0, 0.1).

Every linear, the embedding lookup and the argmax are qlin.h entry points; RMSNorm, rotary embedding
with the KV-cache store and attention are qlin_decoder.h's.  The prompt runs as one batched pass (the
m > 1 matmuls); each decode step is one token at a position held in device memory, so a step can be
captured into a HIP graph and replayed, the argmax writing the next step's token id on the device.
torch provides the device memory and the streams.
"""
from __future__ import annotations

from dataclasses import dataclass

from . import qlin

Q8_0 = 8
QK8_0 = 32


@dataclass
class Qwen2Config:
    layers: int = 24
    hidden: int = 896
    n_heads: int = 14
    kv_heads: int = 2
    head_dim: int = 64
    ffn: int = 4864
    vocab: int = 151936
    eps: float = 1e-6
    theta: float = 1e6
    wtype: int = Q8_0

    @property
    def q_dim(self) -> int:
        return self.n_heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.kv_heads * self.head_dim


def quantize_q8_0(torch, x):
    """ggml's Q8_0 quantizer (quantize_row_q8_0_ref) of a [rows, cols] f32 tensor: per 32 values
    d = amax / 127 (stored as f16), q = round(x * (1 / d)) with ties away from zero; the packed bytes
    [rows, cols / 32 * 34]."""
    rows, cols = x.shape
    xb = x.view(rows, cols // QK8_0, QK8_0)
    d = xb.abs().amax(-1) / 127.0
    inv = torch.where(d > 0, 1.0 / d, torch.zeros_like(d))
    v = xb * inv.unsqueeze(-1)
    q = (torch.sign(v) * torch.floor(v.abs() + 0.5)).to(torch.int8)
    out = torch.empty(rows, cols // QK8_0, 2 + QK8_0, dtype=torch.uint8, device=x.device)
    out[:, :, 0:2] = d.to(torch.float16).view(torch.uint8).view(rows, cols // QK8_0, 2)
    out[:, :, 2:] = q.view(torch.uint8)
    return out.view(rows, -1)


def make_weights(torch, cfg: Qwen2Config, seed: int) -> dict:
    """Random-init weights on the GPU: {'layers': [{wq, wk, wv, wo, wg, wu, wd, attn_norm,
    ffn_norm}], 'final_norm', 'table'}; linears packed Q8_0 (uint8), norms as bf16 bit patterns
    (int16 tensors)."""
    assert cfg.wtype == Q8_0
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)

    def linear(n, k):
        return quantize_q8_0(torch, torch.randn(n, k, device="cuda", generator=gen) * 0.02).contiguous()

    def norm():
        w = (1.0 + 0.1 * torch.randn(cfg.hidden, device="cuda", generator=gen)).to(torch.bfloat16)
        return w.view(torch.int16).contiguous()

    H, F = cfg.hidden, cfg.ffn
    layers = []
    for _ in range(cfg.layers):
        layers.append({"wq": linear(cfg.q_dim, H), "wk": linear(cfg.kv_dim, H), "wv": linear(cfg.kv_dim, H),
                       "wo": linear(H, cfg.q_dim), "wg": linear(F, H), "wu": linear(F, H), "wd": linear(H, F),
                       "attn_norm": norm(), "ffn_norm": norm()})
    return {"layers": layers, "final_norm": norm(), "table": linear(cfg.vocab, H)}


class Qwen2Decoder:
    """Greedy decoding of one sequence; buffers for prompts of up to max_prompt tokens and max_seq
    positions in all."""

    def __init__(self, torch, cfg: Qwen2Config, weights: dict, max_seq: int = 512, max_prompt: int = 64,
                 fuse: bool = True):
        self.torch, self.cfg, self.w = torch, cfg, weights
        self.max_seq, self.max_prompt = max_seq, max_prompt
        # decode steps: each RMSNorm inside the launch of the linear that consumes it (the matrix-core
        # decode kernels take in_dim in whole 128-weight chunks for Q8_0), and the rotary embedding with
        # the cache store inside the attention launch
        self.fuse = fuse and cfg.hidden % 128 == 0
        dev, f32, i32 = "cuda", torch.float32, torch.int32
        H, F, P = cfg.hidden, cfg.ffn, max_prompt
        self.rb_h = qlin.row_bytes(cfg.wtype, H)
        self.rb_q = qlin.row_bytes(cfg.wtype, cfg.q_dim)
        self.rb_f = qlin.row_bytes(cfg.wtype, F)
        self.h = torch.zeros(P, H, dtype=f32, device=dev)        # residual stream
        self.xn = torch.zeros(P, H, dtype=f32, device=dev)
        self.q = torch.zeros(P, cfg.q_dim, dtype=f32, device=dev)
        self.k = torch.zeros(P, cfg.kv_dim, dtype=f32, device=dev)
        self.v = torch.zeros(P, cfg.kv_dim, dtype=f32, device=dev)
        self.attn = torch.zeros(P, cfg.q_dim, dtype=f32, device=dev)
        self.act = torch.zeros(P, F, dtype=f32, device=dev)
        self.logits = torch.zeros(cfg.vocab, dtype=f32, device=dev)
        self.pick_scratch = torch.zeros(8192, dtype=torch.uint8, device=dev)  # the head's per-workgroup picks
        self.kc = [torch.zeros(max_seq, cfg.kv_dim, dtype=f32, device=dev) for _ in range(cfg.layers)]
        self.vc = [torch.zeros(max_seq, cfg.kv_dim, dtype=f32, device=dev) for _ in range(cfg.layers)]
        self.prompt_ids = torch.zeros(P, dtype=i32, device=dev)
        self.token = torch.zeros(1, dtype=i32, device=dev)      # the next step's input token
        self.pos = torch.zeros(1, dtype=i32, device=dev)        # the next step's position
        self.zero = torch.zeros(1, dtype=i32, device=dev)
        self.L = qlin.lib()

    # ---- the calls -------------------------------------------------------------------------------

    def _ok(self, name, rc):
        if rc != 0:
            raise qlin.QlinError(name, rc)

    def _norm(self, x, out, w, rows):
        c = self.cfg
        self._ok("rms_norm", self.L.qlin_launch_rms_norm(x, out, w.data_ptr(), 0, rows, c.hidden, c.eps, 0))

    def _layers(self, rows: int, pos_ptr: int):
        """The decoder layers over `rows` tokens whose first position is *pos_ptr."""
        c, L, t = self.cfg, self.L, c_ptr
        H, F, QD, KD = c.hidden, c.ffn, c.q_dim, c.kv_dim
        h, xn, q, k, v, attn, act = (t(self.h), t(self.xn), t(self.q), t(self.k), t(self.v), t(self.attn),
                                     t(self.act))
        fuse = rows == 1 and self.fuse
        for i, W in enumerate(self.w["layers"]):
            if fuse:
                qlin.rms_norm_quant_gemv_multi(c.wtype, [W["wq"], W["wk"], W["wv"]], self.rb_h, h, W["attn_norm"], 0,
                                               c.eps, 0, [q, k, v], [QD, KD, KD], H)
            elif rows == 1:
                self._norm(h, xn, W["attn_norm"], rows)
                qlin.quant_gemv_multi(c.wtype, [W["wq"], W["wk"], W["wv"]], self.rb_h, xn, [q, k, v], [QD, KD, KD], H)
            else:
                self._norm(h, xn, W["attn_norm"], rows)
                for name, y, n in (("wq", q, QD), ("wk", k, KD), ("wv", v, KD)):
                    self._ok("matmul", L.qlin_launch_quant_matmul(c.wtype, t(W[name]), self.rb_h, xn, y, n, H, rows))
            if fuse:
                self._ok("rope_attend", L.qlin_launch_rope_attend(q, k, v, t(self.kc[i]), t(self.vc[i]), attn,
                                                                  c.n_heads, c.kv_heads, c.head_dim, self.max_seq,
                                                                  pos_ptr, c.theta))
            else:
                self._ok("rope", L.qlin_launch_rope_store_kv(q, k, v, t(self.kc[i]), t(self.vc[i]), rows, c.n_heads,
                                                             c.kv_heads, c.head_dim, self.max_seq, pos_ptr, c.theta))
                self._ok("attend", L.qlin_launch_attend(q, t(self.kc[i]), t(self.vc[i]), attn, rows, c.n_heads,
                                                        c.kv_heads, c.head_dim, self.max_seq, pos_ptr))
            self._ok("o", L.qlin_launch_quant_matmul_add(c.wtype, t(W["wo"]), self.rb_q, attn, h, H, QD, rows))
            if fuse:
                self._ok("norm_swiglu", L.qlin_launch_rms_norm_quant_swiglu(c.wtype, t(W["wg"]), t(W["wu"]), self.rb_h,
                                                                            h, t(W["ffn_norm"]), 0, c.eps, 0, act, F,
                                                                            H))
            elif rows == 1:
                self._norm(h, xn, W["ffn_norm"], rows)
                self._ok("swiglu", L.qlin_launch_quant_swiglu(c.wtype, t(W["wg"]), t(W["wu"]), self.rb_h, self.rb_h,
                                                              xn, act, F, H))
            else:
                self._norm(h, xn, W["ffn_norm"], rows)
                self._ok("swiglu", L.qlin_launch_quant_swiglu_rows(c.wtype, t(W["wg"]), t(W["wu"]), self.rb_h,
                                                                   self.rb_h, xn, act, F, H, rows))
            self._ok("down", L.qlin_launch_quant_matmul_add(c.wtype, t(W["wd"]), self.rb_f, act, h, H, F, rows))

    def _head(self, row: int):
        """Final norm of residual row `row`, the tied output head, and the greedy pick into token."""
        c, L, t = self.cfg, self.L, c_ptr
        hr = t(self.h) + 4 * row * c.hidden
        if self.fuse and hr % 16 == 0:
            # the norm inside the head GEMV, and each of its workgroups' greedy pick in its epilogue (one
            # small launch reduces the picks): two launches instead of norm, GEMV and a scan of every logit
            self._ok("lm_head_argmax", L.qlin_launch_quant_gemv_argmax(
                c.wtype, t(self.w["table"]), self.rb_h, hr, t(self.w["final_norm"]), 0, c.eps, 0, t(self.logits),
                c.vocab, c.hidden, t(self.pick_scratch), t(self.token)))
            return
        self._norm(hr, t(self.xn), self.w["final_norm"], 1)
        self._ok("lm_head", L.qlin_launch_quant_gemv(c.wtype, t(self.w["table"]), self.rb_h, t(self.xn),
                                                     t(self.logits), c.vocab, c.hidden, 1))
        self._ok("argmax", L.qlin_launch_argmax(t(self.logits), c.vocab, t(self.token)))

    def prefill(self, prompt) -> None:
        """The prompt (device int32 tensor of n <= max_prompt ids) at positions 0..n-1 in one batched
        pass; leaves the last position's logits, the greedy token and pos = n."""
        c, t = self.cfg, c_ptr
        n = int(prompt.numel())
        assert 0 < n <= self.max_prompt and n <= self.max_seq
        qlin.set_stream(self.torch.cuda.current_stream())
        self.prompt_ids[:n].copy_(prompt)
        self._ok("embedding", self.L.qlin_launch_quant_embedding(c.wtype, t(self.prompt_ids), t(self.h),
                                                                 t(self.w["table"]), self.rb_h, c.hidden, n))
        self._layers(n, t(self.zero))
        self._head(n - 1)
        self.pos.fill_(n)

    def step(self) -> None:
        """One decode token: the token id and position held on the device; leaves the logits, the next
        greedy token and pos + 1 (no host synchronisation, so a HIP graph can hold it)."""
        c, t = self.cfg, c_ptr
        qlin.set_stream(self.torch.cuda.current_stream())
        self._ok("embedding", self.L.qlin_launch_quant_embedding(c.wtype, t(self.token), t(self.h),
                                                                 t(self.w["table"]), self.rb_h, c.hidden, 1))
        self._layers(1, t(self.pos))
        self._head(0)
        self.pos.add_(1)

    def generate(self, prompt, n_new: int, logits_out=None):
        """Greedy decode of n_new tokens after the prompt, eagerly; returns the token ids (host list).
        logits_out ([n_new, vocab] device tensor, optional) receives each new token's logits."""
        torch = self.torch
        toks = torch.zeros(n_new, dtype=torch.int32, device="cuda")
        self.prefill(prompt)
        for i in range(n_new):
            if i:
                self.step()
            toks[i:i + 1].copy_(self.token)
            if logits_out is not None:
                logits_out[i].copy_(self.logits)
        return toks.cpu().tolist()


def c_ptr(t) -> int:
    return t.data_ptr()
