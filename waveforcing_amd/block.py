"""The Wan attention block on the quantized HIP path, for one chunk on one GPU.

Restates CausalWanAttentionBlock.forward
(naive_rt/rolling_forcing/wan/modules/causal_model.py:349-402), the naive_rt
counterpart of the block WaveRT's SGLang model runs (SGLang is not vendored), with:

* every block linear W8A8 int8 (the ``scope=all`` swap of
  wave_rt/runtime/fp8.py:93-137, per-token / per-channel int8);
* norm + modulation + activation quantization fused into one row kernel;
* q RMSNorm + 3-D RoPE fused into one row kernel; K's RMSNorm + RoPE + FP8
  pack and V's pack fused into another, straight from the QKV output;
* self-attention over the FP8 paged context: this chunk's K/V are packed
  into its pages, then attention reads the prior chunks' pages plus its own
  (the single-GPU form of the paged exchange, paged.py:206-247);
* text cross-attention over the cached 512-token K/V (crossattn_cache,
  model.py:174-183) in the dense-bf16 variant of the attention kernel;
* GELU(tanh) of fc_in's output fused into fc_out's input quantization; gated
  residuals in bf16.

Every step is a HIP kernel from libwf_mi355x.so; torch only allocates and
slices tensors.
"""

from __future__ import annotations

from dataclasses import dataclass, fields

import torch

from . import _lib, rope
from .backend import attn_dense_bf16, paged_attention
from .fp8 import _quant_rows_i8, gemm_i8
from .kv import Fp8PagePool, PagedKV, PageTable

# Wan2.1 shapes (wave_rt/runtime/dummy_model.py:25-35)
PRESETS = {
    "1.3b": dict(dim=1536, heads=12, ffn_dim=8960, layers=30),
    "14b": dict(dim=5120, heads=40, ffn_dim=13824, layers=40),
}
EPS = 1e-6


@dataclass
class BlockParams:
    """bf16 parameters of one attention block (nn.Linear layout [out, in])."""

    modulation: torch.Tensor  # [1, 6, dim]
    q_w: torch.Tensor
    q_b: torch.Tensor
    k_w: torch.Tensor
    k_b: torch.Tensor
    v_w: torch.Tensor
    v_b: torch.Tensor
    o_w: torch.Tensor
    o_b: torch.Tensor
    norm_q: torch.Tensor
    norm_k: torch.Tensor
    norm3_w: torch.Tensor
    norm3_b: torch.Tensor
    cq_w: torch.Tensor
    cq_b: torch.Tensor
    ck_w: torch.Tensor
    ck_b: torch.Tensor
    cv_w: torch.Tensor
    cv_b: torch.Tensor
    co_w: torch.Tensor
    co_b: torch.Tensor
    cnorm_q: torch.Tensor
    cnorm_k: torch.Tensor
    fc_in_w: torch.Tensor
    fc_in_b: torch.Tensor
    fc_out_w: torch.Tensor
    fc_out_b: torch.Tensor

    @property
    def dim(self) -> int:
        return self.q_w.shape[0]

    def to(self, device) -> "BlockParams":
        return BlockParams(**{f.name: getattr(self, f.name).to(device) for f in fields(self)})


def random_block_params(dim: int, ffn_dim: int, seed: int = 0, w_std: float = 0.02, device="cpu") -> BlockParams:
    """Seeded random-init block (bf16): linears ~ N(0, w_std), biases ~ N(0, 0.01), norm weights
    ~ 1 + N(0, 0.05), modulation ~ N(0, 1) / sqrt(dim) (causal_model.py:347).  Drawn on ``device``
    by that device's generator (the CPU and GPU draws of one seed differ)."""
    g = torch.Generator(device=device).manual_seed(seed)

    def lin(o, i):
        return (torch.randn((o, i), generator=g, device=device) * w_std).to(torch.bfloat16)

    def vec(n, std=0.01, mean=0.0):
        return (torch.randn((n,), generator=g, device=device) * std + mean).to(torch.bfloat16)

    return BlockParams(
        modulation=(torch.randn((1, 6, dim), generator=g, device=device) / dim ** 0.5).to(torch.bfloat16),
        q_w=lin(dim, dim), q_b=vec(dim), k_w=lin(dim, dim), k_b=vec(dim), v_w=lin(dim, dim), v_b=vec(dim),
        o_w=lin(dim, dim), o_b=vec(dim), norm_q=vec(dim, 0.05, 1.0), norm_k=vec(dim, 0.05, 1.0),
        norm3_w=vec(dim, 0.05, 1.0), norm3_b=vec(dim),
        cq_w=lin(dim, dim), cq_b=vec(dim), ck_w=lin(dim, dim), ck_b=vec(dim), cv_w=lin(dim, dim), cv_b=vec(dim),
        co_w=lin(dim, dim), co_b=vec(dim), cnorm_q=vec(dim, 0.05, 1.0), cnorm_k=vec(dim, 0.05, 1.0),
        fc_in_w=lin(ffn_dim, dim), fc_in_b=vec(ffn_dim), fc_out_w=lin(dim, ffn_dim), fc_out_b=vec(dim),
    )


@dataclass
class QLinear:
    """Pre-quantized int8 weight [out, in] with per-channel scales and bf16 bias."""

    w: torch.Tensor
    s: torch.Tensor
    b: torch.Tensor | None

    @classmethod
    def from_bf16(cls, w: torch.Tensor, b: torch.Tensor | None, device) -> "QLinear":
        qw, sw = _quant_rows_i8(w.to(device).contiguous())
        return cls(qw, sw, None if b is None else b.to(device).contiguous())


def _ln_quant(x, dim, frame_tokens, q, qs, out=None, w=None, b=None, shift=None, scale=None, res_y=None,
              res_gate=None):
    """LayerNorm (+affine, +modulation) and per-token int8 quant of x, optionally after the residual
    x += res_y (* res_gate) applied in place.  shift/scale/res_gate are frame-row views that share
    one row stride (columns of the modulation tensor)."""
    T = x.shape[0]
    mods = [t for t in (shift, scale, res_gate) if t is not None]
    ld_mod = mods[0].stride(0) if mods else 0
    if any(t.stride(0) != ld_mod or t.stride(-1) != 1 for t in mods):
        raise ValueError("modulation rows must share one row stride with unit column stride")
    _lib.call("wf_gate_residual_ln_quant", x.data_ptr(), T, dim, x.stride(0), _lib.ptr(res_y),
              res_y.stride(0) if res_y is not None else 0, _lib.ptr(res_gate), ld_mod, EPS, _lib.ptr(w),
              _lib.ptr(b), _lib.ptr(shift), _lib.ptr(scale), ld_mod, frame_tokens, _lib.ptr(out),
              out.stride(0) if out is not None else 0, _lib.ptr(q), _lib.ptr(qs), _lib.stream_handle(x.device))


def _rmsnorm_rope(x, head_dim, w, cos, sin, out):
    T, dim = x.shape
    _lib.call("wf_rmsnorm_rope", x.data_ptr(), T, dim, x.stride(0), head_dim, EPS, w.data_ptr(), _lib.ptr(cos),
              _lib.ptr(sin), out.data_ptr(), out.stride(0), _lib.stream_handle(x.device))


def _gate_residual(x, y, gate, frame_tokens):
    T, dim = x.shape
    _lib.call("wf_gate_residual", x.data_ptr(), x.stride(0), y.data_ptr(), y.stride(0), _lib.ptr(gate),
              gate.stride(0) if gate is not None else 0, T, dim, frame_tokens, _lib.stream_handle(x.device))


def apply_pending_residual(x: torch.Tensor, pending, frame_tokens: int) -> torch.Tensor:
    """x = bf16(x + bf16(y * gate)) in place for the (y, gate) a block's forward(defer_residual=True)
    returned: the block's last gated residual (causal_model.py:397-398)."""
    y, gate = pending
    _gate_residual(x, y, gate, frame_tokens)
    return x


def _linear_i8(x, lin: QLinear, ws_q, ws_s, out, gelu=False, gelu_input=False):
    """W8A8 linear of bf16 x [M, K] into out [M, N] via the fused C entry point; ``gelu`` applies GELU(tanh) to
    the output, ``gelu_input`` to x before its quantization."""
    M, K = x.shape
    N = lin.w.shape[0]
    flags = (_lib.GEMM_GELU_TANH if gelu else 0) | (_lib.LINEAR_GELU_INPUT if gelu_input else 0)
    _lib.call("wf_w8a8_linear", x.data_ptr(), M, K, x.stride(0), lin.w.data_ptr(), lin.s.data_ptr(),
              _lib.ptr(lin.b), N, out.data_ptr(), out.stride(0), flags,
              ws_q.data_ptr(), ws_s.data_ptr(), _lib.stream_handle(x.device))
    return out


class QuantizedWanBlock:
    """One Wan block with quantized weights resident on the GPU."""

    def __init__(self, params: BlockParams, heads: int, device="cuda") -> None:
        self.device = torch.device(device)
        self.dim = params.dim
        self.heads = heads
        self.head_dim = self.dim // heads
        self.ffn_dim = params.fc_in_w.shape[0]
        dev = self.device
        self.modulation = params.modulation.to(dev)
        self.qkv = QLinear.from_bf16(torch.cat([params.q_w, params.k_w, params.v_w], 0),
                                     torch.cat([params.q_b, params.k_b, params.v_b], 0), dev)
        self.o = QLinear.from_bf16(params.o_w, params.o_b, dev)
        self.cq = QLinear.from_bf16(params.cq_w, params.cq_b, dev)
        self.ck = QLinear.from_bf16(params.ck_w, params.ck_b, dev)
        self.cv = QLinear.from_bf16(params.cv_w, params.cv_b, dev)
        self.co = QLinear.from_bf16(params.co_w, params.co_b, dev)
        self.fc_in = QLinear.from_bf16(params.fc_in_w, params.fc_in_b, dev)
        self.fc_out = QLinear.from_bf16(params.fc_out_w, params.fc_out_b, dev)
        self.norm_q = params.norm_q.to(dev)
        self.norm_k = params.norm_k.to(dev)
        self.norm3_w = params.norm3_w.to(dev)
        self.norm3_b = params.norm3_b.to(dev)
        self.cnorm_q = params.cnorm_q.to(dev)
        self.cnorm_k = params.cnorm_k.to(dev)
        self._ws: dict = {}

    @classmethod
    def from_packed(cls, packed: dict, heads: int, device="cuda") -> "QuantizedWanBlock":
        """A block from offline-packed tensors (waveforcing_amd.checkpoint.pack_block /
        load_packed): int8 weights and scales go to the GPU as they are, nothing is quantized."""
        self = cls.__new__(cls)
        dev = self.device = torch.device(device)

        def lin(name):
            b = packed.get(f"{name}_b")
            return QLinear(packed[f"{name}_i8"].to(dev).contiguous(), packed[f"{name}_scale"].to(dev).contiguous(),
                           None if b is None else b.to(dev).contiguous())

        q, k, v = lin("q"), lin("k"), lin("v")
        self.qkv = QLinear(torch.cat([q.w, k.w, v.w], 0), torch.cat([q.s, k.s, v.s], 0),
                           torch.cat([q.b, k.b, v.b], 0))
        self.o, self.cq, self.ck, self.cv, self.co = lin("o"), lin("cq"), lin("ck"), lin("cv"), lin("co")
        self.fc_in, self.fc_out = lin("fc_in"), lin("fc_out")
        self.dim = self.qkv.w.shape[1]
        self.heads = heads
        self.head_dim = self.dim // heads
        self.ffn_dim = self.fc_in.w.shape[0]
        for name in ("modulation", "norm_q", "norm_k", "norm3_w", "norm3_b", "cnorm_q", "cnorm_k"):
            setattr(self, name, packed[name].to(dev).contiguous())
        self._ws = {}
        return self

    # -- workspace (allocated once per token count; the kernels never allocate)
    def share_workspace(self, other: "QuantizedWanBlock") -> None:
        """Use other's activation buffers (blocks of one shape that never run concurrently)."""
        if (self.dim, self.ffn_dim, self.device) != (other.dim, other.ffn_dim, other.device):
            raise ValueError("only blocks of the same shape and device can share a workspace")
        self._ws = other._ws

    def new_workspace(self, T: int) -> dict:
        """Activation buffers of one forward over T tokens (any block of this shape can use them)."""
        dev, dim = self.device, self.dim
        bf = dict(dtype=torch.bfloat16, device=dev)
        qbuf = torch.empty((T * max(dim, self.ffn_dim),), dtype=torch.int8, device=dev)
        return dict(
            T=T, aq=qbuf[:T * dim].view(T, dim), fq=qbuf[:T * self.ffn_dim].view(T, self.ffn_dim),
            as_=torch.empty((T,), dtype=torch.float32, device=dev),
            qkv=torch.empty((T, 3 * dim), **bf), attn=torch.empty((T, dim), **bf), y=torch.empty((T, dim), **bf),
            cq=torch.empty((T, dim), **bf), ffn=torch.empty((T, self.ffn_dim), **bf),
        )

    def _workspace(self, T: int) -> dict:
        ws = self._ws.get(T)
        if ws is None:
            ws = self._ws[T] = self.new_workspace(T)
        return ws

    def text_kv(self, context: torch.Tensor):
        """Cross-attention K/V of the text context [L, dim] (computed once per request)."""
        L = context.shape[0]
        dev = self.device
        ws_q = torch.empty((L, self.dim), dtype=torch.int8, device=dev)
        ws_s = torch.empty((L,), dtype=torch.float32, device=dev)
        k = torch.empty((L, self.dim), dtype=torch.bfloat16, device=dev)
        v = torch.empty((L, self.dim), dtype=torch.bfloat16, device=dev)
        _linear_i8(context, self.ck, ws_q, ws_s, k)
        kn = torch.empty_like(k)
        _rmsnorm_rope(k, self.head_dim, self.cnorm_k, None, None, kn)
        _linear_i8(context, self.cv, ws_q, ws_s, v)
        return kn.view(L, self.heads, self.head_dim), v.view(L, self.heads, self.head_dim)

    def forward(self, x: torch.Tensor, e: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, pool: Fp8PagePool,
                context_table: PageTable, own_table: PageTable, n_context: int, text_kv,
                unroped_k_out: torch.Tensor | None = None, es: torch.Tensor | None = None, pending=None,
                defer_residual: bool = False, ws: dict | None = None, kv_only: bool = False):
        """Advance x [T, dim] bf16 in place through the block.

        e: [F, 6, dim] bf16 time modulation of the chunk's F frames.
        cos/sin: RoPE tables [T, head_dim/2] of this chunk.
        pool/context_table/n_context: this layer's FP8 page context (prior
        chunks' pages followed by ``own_table``'s pages), of n_context keys
        including this chunk's T tokens, which are packed into own_table here.
        unroped_k_out: optional [T, dim] bf16 buffer for this chunk's normalized,
        un-rotated K (the exchange's unroped_key, kept for the anchor re-RoPE).
        es: optional precomputed bf16 ``modulation + e`` [F, 6, dim] of this block
        (a stack adds every layer's table in one launch).
        pending: optional (y, gate) residual left by the previous block's
        ``defer_residual``; it is applied in front of this block's first
        LayerNorm, in the same kernel, with the same arithmetic as a separate
        wf_gate_residual.
        defer_residual: leave this block's last gated residual undone and return
        (x, (y, gate)) for the next block (or apply_pending_residual); y is this
        block's workspace, valid until the next forward of a block sharing it
        has run its first LayerNorm.
        ws: optional activation buffers from :meth:`new_workspace` (passes that run
        concurrently on different streams each bring their own); default: the
        block's own, shared with the blocks of its stack.
        kv_only: stop once this chunk's K and V are in its pages (and the
        un-rotated K in ``unroped_k_out``), for a pass whose output nobody reads;
        x then holds the block's input with ``pending`` applied, and (x, None)
        is returned.
        """
        T, dim = x.shape
        F = e.shape[0]
        if T % F:
            raise ValueError(f"{T} tokens do not split into {F} frames")
        ft = T // F
        H, hd = self.heads, self.head_dim
        if ws is None:
            ws = self._workspace(T)
        elif ws["T"] != T or ws["qkv"].shape[1] != 3 * dim or ws["ffn"].shape[1] != self.ffn_dim:
            raise ValueError(f"workspace for {ws['T']} tokens of another shape given to a {T}-token forward")
        # e = (modulation + e).chunk(6)  (causal_model.py:376), bf16: one add; the kernels read
        # the six [F, dim] chunks as strided frame rows of it.
        if es is None:
            es = self.modulation[0].unsqueeze(0) + e
        elif es.shape != (F, 6, dim):
            raise ValueError(f"es must be [{F}, 6, {dim}], got {tuple(es.shape)}")
        e0, e1, e2, e3, e4, e5 = (es[:, i] for i in range(6))
        aq, as_ = ws["aq"], ws["as_"]

        # self-attention: LN1 + modulation + int8 quant -> fused QKV
        if pending is None:
            _ln_quant(x, dim, ft, aq, as_, shift=e0, scale=e1)
        else:  # the previous block's last gated residual, fused in front of LN1
            _ln_quant(x, dim, ft, aq, as_, shift=e0, scale=e1, res_y=pending[0], res_gate=pending[1])
        gemm_i8(aq, self.qkv.w, as_, self.qkv.s, self.qkv.b, out=ws["qkv"])
        qkv = ws["qkv"]
        q, k, v = qkv[:, :dim], qkv[:, dim:2 * dim], qkv[:, 2 * dim:]
        # q and K: RMSNorm + RoPE in one pass (q in place: each row is read whole before it is
        # written), K FP8-packed into this chunk's pages and V packed beside it
        if kv_only:
            pool.pack_k_norm_rope(k, v, own_table, self.norm_k, EPS, (cos, sin), ku_out=unroped_k_out)
            return x, None
        pool.pack_k_norm_rope(k, v, own_table, self.norm_k, EPS, (cos, sin), ku_out=unroped_k_out, q=q,
                              norm_q=self.norm_q)
        ctx = PagedKV(pool, context_table, n_context)
        paged_attention()(q.view(T, H, hd), ctx, out=ws["attn"].view(T, H, hd))
        _linear_i8(ws["attn"], self.o, aq, as_, ws["y"])

        # gated residual + norm3 (affine) + quant -> q, RMSNorm, attention over text, o
        _ln_quant(x, dim, ft, aq, as_, w=self.norm3_w, b=self.norm3_b, res_y=ws["y"], res_gate=e2)
        gemm_i8(aq, self.cq.w, as_, self.cq.s, self.cq.b, out=ws["y"])
        _rmsnorm_rope(ws["y"], hd, self.cnorm_q, None, None, ws["cq"])
        tk, tv = text_kv
        attn_dense_bf16(ws["cq"].view(T, H, hd), tk, tv, out=ws["attn"].view(T, H, hd))
        _linear_i8(ws["attn"], self.co, aq, as_, ws["y"])

        # residual + LN2 + modulation + quant -> fc_in -> GELU + quant -> fc_out: the GELU(tanh) of fc_in's bf16
        # output runs in fc_out's input quantizer (the same values the GEMM epilogue would store)
        _ln_quant(x, dim, ft, aq, as_, shift=e3, scale=e4, res_y=ws["y"])
        gemm_i8(aq, self.fc_in.w, as_, self.fc_in.s, self.fc_in.b, out=ws["ffn"])
        _linear_i8(ws["ffn"], self.fc_out, ws["fq"], as_, ws["y"], gelu_input=True)
        if defer_residual:
            return x, (ws["y"], e5)
        _gate_residual(x, ws["y"], e5, ft)
        return x
