"""End-to-end decode stand-in for the benchmark's config 4 (Qwen3-8B greedy decode): a random-init
Qwen3-architecture decoder whose every weight product runs through the
quantized matrix-product library (libstark_qmm: 4-bit MLX-affine layer
projections, an 8-bit lm_head), with the decode-step kernels of
libstark_decode around them (RMSNorm, per-head q/k norm + RoPE + KV write,
GQA flash-decoding attention over a bf16 cache, gated SiLU, greedy argmax).

A token step is one fixed sequence of launches that reads the position from
device memory, so it is captured once in a HIP graph and replayed per token.

Not a Stark component: Stark's own decoder is its Rust model runtime
(crates/stark-engine/src/encodable_block/transformer_layer.rs). This module
exists to measure tokens/s of the quantized path in a real decode loop.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass
from typing import Optional

import torch

from . import qmm as Q

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(HERE, "libstark_decode.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is not built (run __graft_entry__.build())")
        L = C.CDLL(path)
        vp, u32, f32, ip = C.c_void_p, C.c_uint32, C.c_float, C.c_void_p
        L.stark_decode_rms_norm.argtypes = [vp, vp, vp, u32, f32, vp]
        L.stark_decode_qk_norm_rope.argtypes = [vp, vp, vp, vp, vp, vp, vp, ip, u32, u32, u32, f32, f32, vp]
        L.stark_decode_attn_chunks.argtypes = [u32]
        L.stark_decode_attn_chunks.restype = u32
        L.stark_decode_attention.argtypes = [vp, vp, vp, vp, vp, vp, ip, u32, u32, u32, vp]
        L.stark_decode_attention_fused.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, ip, u32, u32, u32,
                                                   f32, f32, vp]
        L.stark_decode_silu_mul.argtypes = [vp, vp, vp, u32, vp]
        L.stark_decode_argmax.argtypes = [vp, u32, ip, ip, ip, u32, vp]
        L.stark_decode_embed.argtypes = [vp, ip, vp, u32, u32, vp]
        L.stark_decode_embed_tagged.argtypes = [vp, ip, vp, u32, u32, u32, ip, vp]
        L.stark_decode_untag.argtypes = [vp, vp, u32, vp]
        _LIB = L
    return _LIB


def _ok(st, what):
    if st != 0:
        raise RuntimeError(f"{what}: status {st}")


@dataclass
class Qwen3Config:
    hidden: int = 4096
    layers: int = 36
    q_heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    intermediate: int = 12288
    vocab: int = 151936
    eps: float = 1e-6
    rope_theta: float = 1e6
    group: int = 64


def quantize_affine_gpu(w: torch.Tensor, bits: int = 4, group: int = 64):
    """MLX affine quantization: per group scale = (max - min)/(2^bits - 1)
    and bias = min as bf16, q = clamp(round((w - bias)/scale)); codes
    little-endian (low nibble first for 4-bit); planes in the converter's
    group-output layout [G][N] (N % 4 == 0). Returns (codes u8, scales, biases)
    with the planes as int16 bit patterns."""
    n, k = w.shape
    g = w.view(n, k // group, group)
    mn, mx = g.amin(dim=2), g.amax(dim=2)
    levels = (1 << bits) - 1
    s = ((mx - mn) / float(levels)).to(torch.bfloat16)
    b = mn.to(torch.bfloat16)
    sf, bf = s.float().unsqueeze(2), b.float().unsqueeze(2)
    q = torch.where(sf > 0, torch.round((g - bf) / torch.where(sf > 0, sf, torch.ones_like(sf))),
                    torch.zeros_like(g)).clamp(0, levels).to(torch.uint8).view(n, k)
    codes = (q[:, 0::2] | (q[:, 1::2] << 4)).contiguous() if bits == 4 else q.contiguous()
    return codes, s.t().contiguous().view(torch.int16), b.t().contiguous().view(torch.int16)


class Qwen3Decoder:
    """Random-init Qwen3-architecture decoder on one GPU (bf16 activations and
    KV cache; weights quantized W4 g64, lm_head W8 g64; embeddings bf16).

    fused: the attention/MLP RMS norms and the gated SiLU run as input
    prologues of the products that read them (stark_qmm_encode_many_prologue;
    bit-identical rows, three launches fewer per layer). None = whenever the
    shapes allow it (hidden and intermediate multiples of 4096).

    In the fused form with intermediate 12288 the down product runs as three
    K slices of one chained launch with plain rows (stark_qmm_encode_chain;
    the twelve-wave launch's sum order, so the same bits, on three times the
    workgroups: 13.6-13.7 -> 12.2 us a layer).

    chain: a layer's products after attention -- o, gate/up, down (K split in
    three slices) and the next layer's q/k/v -- run as ONE chained launch
    (stark_qmm_encode_chain): the residual row and the gate/up rows are kept
    as tagged words (bf16 | tag << 16) through which the stages hand over
    inside the launch. Same rows, bit for bit, as the fused form. None =
    whenever the shapes allow it (hidden 4096 and intermediate a multiple of
    12288); off by default."""

    def __init__(self, cfg: Qwen3Config, capacity: int, seed: int = 0, device: str = "cuda",
                 fused: Optional[bool] = None, chain: bool = False):
        self.cfg, self.cap = cfg, capacity
        H, I, hd = cfg.hidden, cfg.intermediate, cfg.head_dim
        eligible = H % 4096 == 0 and I % 4096 == 0
        if fused and not eligible:
            raise ValueError("the fused prologues need hidden and intermediate sizes that are multiples of 4096")
        self.fused = eligible if fused is None else fused
        chain_ok = self.fused and H == 4096 and I % 12288 == 0 and (cfg.q_heads + 2 * cfg.kv_heads) * hd % 32 == 0
        # the fused form's down product as three K slices of one chained
        # launch (stark_qmm_encode_chain, plain rows): the twelve-wave launch's
        # exact sum order, on three times the workgroups
        self.split_down = self.fused and I == 12288 and H % 32 == 0
        if chain and not chain_ok:
            raise ValueError("the chained launch needs the fused form, hidden 4096 and intermediate a multiple of 12288")
        self.chain = bool(chain)
        qd, kd = cfg.q_heads * hd, cfg.kv_heads * hd
        gen = torch.Generator(device=device)
        gen.manual_seed(seed)
        dev = torch.device(device)

        def randn(*shape, std=0.02):
            return torch.randn(*shape, generator=gen, device=dev) * std

        def qmat(n, k, bits=4):
            codes, s, b = quantize_affine_gpu(randn(n, k), bits, cfg.group)
            return dict(n=n, k=k, bits=bits, codes=codes, scales=s, biases=b)

        def norm_w(n):
            return (1.0 + randn(n, std=0.05)).to(torch.bfloat16)

        self.embed = randn(cfg.vocab, H).to(torch.bfloat16)
        self.layers = []
        for _ in range(cfg.layers):
            self.layers.append(dict(
                attn_norm=norm_w(H), mlp_norm=norm_w(H), q_norm=norm_w(hd), k_norm=norm_w(hd),
                q=qmat(qd, H), k=qmat(kd, H), v=qmat(kd, H), o=qmat(H, qd),
                gate=qmat(I, H), up=qmat(I, H), down=qmat(H, I),
                kcache=torch.zeros(cfg.kv_heads, capacity, hd, dtype=torch.bfloat16, device=dev),
                vcache=torch.zeros(cfg.kv_heads, capacity, hd, dtype=torch.bfloat16, device=dev)))
        self.final_norm = norm_w(H)
        self.lm_head = qmat(cfg.vocab, H, bits=8)
        # activations and scratch
        bf16 = torch.bfloat16
        self.x = torch.zeros(H, dtype=bf16, device=dev)
        self.h = torch.zeros(H, dtype=bf16, device=dev)
        self.q = torch.zeros(qd, dtype=bf16, device=dev)
        self.k = torch.zeros(kd, dtype=bf16, device=dev)
        self.v = torch.zeros(kd, dtype=bf16, device=dev)
        self.attn = torch.zeros(qd, dtype=bf16, device=dev)
        self.g = torch.zeros(I, dtype=bf16, device=dev)
        self.u = torch.zeros(I, dtype=bf16, device=dev)
        self.a = torch.zeros(I, dtype=bf16, device=dev)
        self.logits = torch.zeros(cfg.vocab, dtype=torch.float32, device=dev)
        if self.chain:  # tagged rows of the chained launches
            self.xt = torch.zeros(H, dtype=torch.int32, device=dev)
            self.gt = torch.zeros(I, dtype=torch.int32, device=dev)
            self.ut = torch.zeros(I, dtype=torch.int32, device=dev)
        nch = lib().stark_decode_attn_chunks(capacity)
        self.po = torch.zeros(cfg.q_heads * nch * hd, dtype=torch.float32, device=dev)
        self.pml = torch.zeros(cfg.q_heads * nch * 2, dtype=torch.float32, device=dev)
        self.token = torch.zeros(1, dtype=torch.int32, device=dev)
        self.pos = torch.zeros(1, dtype=torch.int32, device=dev)
        self.history = torch.zeros(capacity + 1, dtype=torch.int32, device=dev)
        self.kern4 = Q.MatmulKernel(Q.BF16, Q.BF16, Q.BF16)
        self.kern_lm = Q.MatmulKernel(Q.BF16, Q.BF16, Q.F32)
        self._prepare()
        self.graph = None

    def _args(self, mat, a, d, accumulate=False):
        return Q.MatmulArguments(
            a=a, m=1, n=mat["n"], k=mat["k"], d=d,
            b=Q.QuantizedB(codes=mat["codes"], scales=mat["scales"], correction_data=mat["biases"],
                           mode=Q.MODE_U4 if mat["bits"] == 4 else Q.MODE_U8, group_size=self.cfg.group,
                           params=Q.QuantParams(Q.GROUP_OUTPUT, mat["n"], mat["k"] // self.cfg.group)),
            d_transform=Q.MatmulDOps(accumulate=accumulate))

    # tags of the chained form: the embedding row, then per layer i the
    # residual after o, the gate/up rows, the residual after down
    TAG_EMBED = 1

    @staticmethod
    def _tags(i):
        return 2 + 3 * i, 3 + 3 * i, 4 + 3 * i

    def _prepare_chain(self):
        K4, eps, L = self.kern4, self.cfg.eps, self.layers
        CP = Q.ChainProduct

        def qkv(layer, in_tag, stage):
            return [CP(self._args(layer[w], self.xt, out), stage, Q.PROLOGUE_RMS_NORM, layer["attn_norm"], eps,
                       in_tag=in_tag) for w, out in (("q", self.q), ("k", self.k), ("v", self.v))]

        self.chain_head = K4.prepare_chain(qkv(L[0], self.TAG_EMBED, 0))
        self.chains = []
        for i, layer in enumerate(L):
            to, tgu, td = self._tags(i)
            prods = [CP(self._args(layer["o"], self.attn, self.xt, accumulate=True), 0, out_tag=to),
                     CP(self._args(layer["gate"], self.xt, self.gt), 1, Q.PROLOGUE_RMS_NORM, layer["mlp_norm"], eps,
                        in_tag=to, out_tag=tgu),
                     CP(self._args(layer["up"], self.xt, self.ut), 1, Q.PROLOGUE_RMS_NORM, layer["mlp_norm"], eps,
                        in_tag=to, out_tag=tgu),
                     CP(self._args(layer["down"], self.gt, self.xt, accumulate=True), 2, Q.PROLOGUE_SILU_GATE, self.ut,
                        in_tag=tgu, out_tag=td, acc_tag=to, k_slices=self.cfg.intermediate // 4096, part_tag=td)]
            if i + 1 < len(L):
                prods += qkv(L[i + 1], td, 3)
            self.chains.append(K4.prepare_chain(prods))
        need = max(c.workspace_bytes for c in self.chains + [self.chain_head])
        self.chain_ws = torch.zeros((need + 7) // 8, dtype=torch.int64, device=self.x.device)

    def chain_status(self) -> int:
        """Non-zero when a wait of a chained launch gave up (rows invalid)."""
        ws = getattr(self, "chain_ws", None)
        return 0 if ws is None else int(ws[0].item() & 0xffffffff)

    def _prepare(self):
        K4 = self.kern4
        self.batches = []
        if self.chain:
            self._prepare_chain()
        if self.fused and self.split_down and not self.chain:
            self.down_chains = [K4.prepare_chain([Q.ChainProduct(
                self._args(L["down"], self.g, self.x, accumulate=True), 0, Q.PROLOGUE_SILU_GATE, self.u,
                k_slices=self.cfg.intermediate // 4096, part_tag=200 + i)]) for i, L in enumerate(self.layers)]
            need = max(c.workspace_bytes for c in self.down_chains)
            self.chain_ws = torch.zeros((need + 7) // 8, dtype=torch.int64, device=self.x.device)
        if self.fused:
            eps = self.cfg.eps
            for L in self.layers:
                self.batches.append(dict(
                    qkv=K4.prepare_many_prologue([self._args(L["q"], self.x, self.q), self._args(L["k"], self.x, self.k),
                                                  self._args(L["v"], self.x, self.v)],
                                                 Q.PROLOGUE_RMS_NORM, L["attn_norm"], eps),
                    o=K4.prepare_many([self._args(L["o"], self.attn, self.x, accumulate=True)]),
                    gu=K4.prepare_many_prologue([self._args(L["gate"], self.x, self.g),
                                                 self._args(L["up"], self.x, self.u)],
                                                Q.PROLOGUE_RMS_NORM, L["mlp_norm"], eps),
                    down=K4.prepare_many_prologue([self._args(L["down"], self.g, self.x, accumulate=True)],
                                                  Q.PROLOGUE_SILU_GATE, self.u)))
            self.lm_batch = self.kern_lm.prepare_many([self._args(self.lm_head, self.h, self.logits)])
            return
        for L in self.layers:
            self.batches.append(dict(
                qkv=K4.prepare_many([self._args(L["q"], self.h, self.q), self._args(L["k"], self.h, self.k),
                                     self._args(L["v"], self.h, self.v)]),
                o=K4.prepare_many([self._args(L["o"], self.attn, self.x, accumulate=True)]),
                gu=K4.prepare_many([self._args(L["gate"], self.h, self.g), self._args(L["up"], self.h, self.u)]),
                down=K4.prepare_many([self._args(L["down"], self.a, self.x, accumulate=True)])))
        self.lm_batch = self.kern_lm.prepare_many([self._args(self.lm_head, self.h, self.logits)])

    def fill_context(self, length: int, seed: int = 1):
        """Synthetic KV for a prompt of `length` tokens (values N(0, 1) in bf16)
        and the position set to `length`; the last prompt token is drawn
        uniformly from the vocabulary."""
        gen = torch.Generator(device=self.x.device)
        gen.manual_seed(seed)
        for L in self.layers:
            L["kcache"][:, :length].normal_(0, 1, generator=gen)
            L["vcache"][:, :length].normal_(0, 1, generator=gen)
        self.pos.fill_(length)
        self.token.fill_(int(torch.randint(0, self.cfg.vocab, (1,), generator=gen, device=self.x.device).item()))

    def step(self, stream=None, trace=None):
        """One greedy token: embed the current token, run every layer at the
        current position, lm_head, argmax; advances the device position.
        trace(layer, stage), when given, is called after each launch (eager
        use only: tests snapshot the activations there)."""
        t = trace if trace is not None else (lambda layer, stage: None)
        cfg, D = self.cfg, lib()
        s = stream if stream is not None else torch.cuda.current_stream()
        sp = C.c_void_p(s.cuda_stream)
        H, I = cfg.hidden, cfg.intermediate
        p = lambda t: C.c_void_p(t.data_ptr())
        if self.chain:
            self._step_chain(D, s, sp, p, t)
            return
        _ok(D.stark_decode_embed(p(self.embed), p(self.token), p(self.x), H, cfg.vocab, sp), "embed")
        t(-1, "embed")
        for i, (L, B) in enumerate(zip(self.layers, self.batches)):
            if not self.fused:  # else the qkv products normalise x as they stage it
                _ok(D.stark_decode_rms_norm(p(self.x), p(L["attn_norm"]), p(self.h), H, cfg.eps, sp), "attn_norm")
                t(i, "attn_norm")
            self.kern4.encode_prepared(B["qkv"], s)
            t(i, "qkv")
            # q/k norm + RoPE, KV write and attention partials in one launch, then the chunk reduction
            _ok(D.stark_decode_attention_fused(p(self.q), p(self.k), p(self.v), p(L["q_norm"]), p(L["k_norm"]),
                                               p(L["kcache"]), p(L["vcache"]), p(self.po), p(self.pml), p(self.attn), p(self.pos), cfg.q_heads, cfg.kv_heads, self.cap,
                                               cfg.rope_theta, cfg.eps, sp), "attention")
            t(i, "attention")
            self.kern4.encode_prepared(B["o"], s)
            t(i, "o")
            if not self.fused:
                _ok(D.stark_decode_rms_norm(p(self.x), p(L["mlp_norm"]), p(self.h), H, cfg.eps, sp), "mlp_norm")
                t(i, "mlp_norm")
            self.kern4.encode_prepared(B["gu"], s)
            t(i, "gate_up")
            if not self.fused:  # else the down product stages silu(g) * u
                _ok(D.stark_decode_silu_mul(p(self.g), p(self.u), p(self.a), I, sp), "silu_mul")
                t(i, "silu_mul")
            if self.fused and self.split_down:
                self.kern4.encode_chain(self.down_chains[i], self.chain_ws, self.pos, s)
            else:
                self.kern4.encode_prepared(B["down"], s)
            t(i, "down")
        _ok(D.stark_decode_rms_norm(p(self.x), p(self.final_norm), p(self.h), H, cfg.eps, sp), "final_norm")
        t(-1, "final_norm")
        self.kern_lm.encode_prepared(self.lm_batch, s)
        t(-1, "lm_head")
        _ok(D.stark_decode_argmax(p(self.logits), cfg.vocab, p(self.token), p(self.pos), p(self.history),
                             self.history.numel(), sp),
            "argmax")

    def _step_chain(self, D, s, sp, p, t):
        """step() of the chained form: embedding (tagged), the first layer's
        q/k/v, then per layer the attention and one chained launch."""
        cfg, H = self.cfg, self.cfg.hidden
        _ok(D.stark_decode_embed_tagged(p(self.embed), p(self.token), p(self.xt), H, cfg.vocab, self.TAG_EMBED,
                                        p(self.pos), sp), "embed")
        t(-1, "embed")
        self.kern4.encode_chain(self.chain_head, self.chain_ws, self.pos, s)
        t(0, "qkv")
        for i, L in enumerate(self.layers):
            _ok(D.stark_decode_attention_fused(p(self.q), p(self.k), p(self.v), p(L["q_norm"]), p(L["k_norm"]),
                                               p(L["kcache"]), p(L["vcache"]), p(self.po), p(self.pml), p(self.attn),
                                               p(self.pos), cfg.q_heads, cfg.kv_heads, self.cap, cfg.rope_theta,
                                               cfg.eps, sp), "attention")
            t(i, "attention")
            self.kern4.encode_chain(self.chains[i], self.chain_ws, self.pos, s)
            t(i, "chain")
        _ok(D.stark_decode_untag(p(self.xt), p(self.x), H, sp), "untag")
        _ok(D.stark_decode_rms_norm(p(self.x), p(self.final_norm), p(self.h), H, cfg.eps, sp), "final_norm")
        t(-1, "final_norm")
        self.kern_lm.encode_prepared(self.lm_batch, s)
        t(-1, "lm_head")
        _ok(D.stark_decode_argmax(p(self.logits), cfg.vocab, p(self.token), p(self.pos), p(self.history),
                                  self.history.numel(), sp), "argmax")

    def capture(self):
        """Capture one token step in a graph (after one eager step has built
        the library's per-shape schedules)."""
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                self.step(s)
        torch.cuda.current_stream().wait_stream(s)
        self.graph = g
        return g


def qmm_untag(words: torch.Tensor) -> torch.Tensor:
    """bf16 values of a tagged row (the chained form's residual row)."""
    return Q.untag_rows(words)[0]
