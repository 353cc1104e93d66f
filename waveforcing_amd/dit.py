"""The Wan DiT around the quantized block stack: one chunk's forward from its noisy latent to x0.

Restates the chunk forward of the wavefront, WaveBackend.forward_chunk
(wave_rt/runtime/backend.py:456-490): the CausalWanModel inference forward
(naive_rt/rolling_forcing/wan/modules/causal_model.py:779-880) for one
3-frame chunk at one denoising step, followed by the flow-matching x0
conversion (wan_wrapper.py:169-193):

* patch embedding: nn.Conv3d(16, dim, kernel = stride = (1, 2, 2))
  (causal_model.py:517-518), as wf_patchify_bf16 + wf_gemm_bf16;
* time embedding sin(t) -> Linear -> SiLU -> Linear and time projection
  SiLU -> Linear(dim, 6 dim) (causal_model.py:522-525,840-844), one timestep
  for every frame of the chunk (backend.py:471-473);
* text embedding Linear(4096, dim) -> GELU(tanh) -> Linear(dim, dim) over
  the context padded to 512 tokens, once per request (:519-521,848-855),
  whose per-layer cross-attention K/V the stack caches;
* the blocks: QuantizedWanStack.run_pass over the paged FP8 exchange;
* head: LayerNorm * (1 + e[1]) + e[0] with e = head modulation + time
  embedding (wf_ln_modulate_quant), Linear(dim, 64) (CausalHead,
  causal_model.py:406-433);
* unpatchify + x0 = xt - sigma * flow in float64
  (wf_unpatchify_flow_x0_bf16), x0 written (B, T, C, H, W).

The reference swaps only the blocks' linears to W8A8 (wave_rt/runtime/
fp8.py:93-137), so these layers stay bf16, on the bf16 matrix cores.  The
sinusoidal table (a few hundred float64 values) is computed on the host.
"""

from __future__ import annotations

from dataclasses import dataclass, fields

import torch

from . import _lib
from .exchange import Pass, TickPlan
from .schedule import FlowMatchSchedule
from .stack import QuantizedWanStack

EPS = 1e-6
IN_DIM = OUT_DIM = 16
TEXT_DIM = 4096
FREQ_DIM = 256
TEXT_LEN = 512


@dataclass
class DiTParams:
    """bf16 parameters of the DiT around the blocks (nn.Linear layout [out, in])."""

    patch_w: torch.Tensor   # [dim, 16, 1, 2, 2]
    patch_b: torch.Tensor
    text1_w: torch.Tensor   # [dim, 4096]
    text1_b: torch.Tensor
    text2_w: torch.Tensor   # [dim, dim]
    text2_b: torch.Tensor
    time1_w: torch.Tensor   # [dim, 256]
    time1_b: torch.Tensor
    time2_w: torch.Tensor   # [dim, dim]
    time2_b: torch.Tensor
    proj_w: torch.Tensor    # [6 dim, dim]
    proj_b: torch.Tensor
    head_mod: torch.Tensor  # [1, 2, dim]
    head_w: torch.Tensor    # [64, dim]
    head_b: torch.Tensor    # [64]

    @property
    def dim(self) -> int:
        return self.patch_w.shape[0]

    def to(self, device) -> "DiTParams":
        return DiTParams(**{f.name: getattr(self, f.name).to(device) for f in fields(self)})


def random_dit_params(dim: int, seed: int = 0, device="cpu", head_std: float = 0.02) -> DiTParams:
    """Seeded random init following CausalWanModel.init_weights (causal_model.py:1105-1127): xavier-uniform
    patch embedding, N(0, 0.02) text and time embeddings, xavier-uniform time projection, head modulation
    N(0, 1) / sqrt(dim) (:420).  Biases are drawn N(0, 0.01) instead of zero and the head weight N(0, head_std)
    instead of zero, so that every bias and the blocks' output reach the result."""
    g = torch.Generator(device=device).manual_seed(seed)

    def normal(shape, std):
        return (torch.randn(shape, generator=g, device=device) * std).to(torch.bfloat16)

    def xavier(out_f, in_f, shape=None):
        bound = (6.0 / (in_f + out_f)) ** 0.5
        w = (torch.rand((out_f, in_f), generator=g, device=device) * 2 - 1) * bound
        return w.reshape(shape if shape is not None else (out_f, in_f)).to(torch.bfloat16)

    return DiTParams(
        patch_w=xavier(dim, IN_DIM * 4, (dim, IN_DIM, 1, 2, 2)), patch_b=normal((dim,), 0.01),
        text1_w=normal((dim, TEXT_DIM), 0.02), text1_b=normal((dim,), 0.01),
        text2_w=normal((dim, dim), 0.02), text2_b=normal((dim,), 0.01),
        time1_w=normal((dim, FREQ_DIM), 0.02), time1_b=normal((dim,), 0.01),
        time2_w=normal((dim, dim), 0.02), time2_b=normal((dim,), 0.01),
        proj_w=xavier(6 * dim, dim), proj_b=normal((6 * dim,), 0.01),
        head_mod=normal((1, 2, dim), dim ** -0.5), head_w=normal((OUT_DIM * 4, dim), head_std),
        head_b=normal((OUT_DIM * 4,), 0.01),
    )


def sinusoidal_embedding(t: float, frames: int, dim: int = FREQ_DIM) -> torch.Tensor:
    """sinusoidal_embedding_1d (model.py:15-26) of one timestep for every frame, float64 [frames, dim]."""
    half = dim // 2
    pos = torch.full((frames,), float(t), dtype=torch.float64)
    sinusoid = torch.outer(pos, torch.pow(10000, -torch.arange(half).to(pos).div(half)))
    return torch.cat([torch.cos(sinusoid), torch.sin(sinusoid)], dim=1)


def gemm_bf16(a: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None, out: torch.Tensor | None = None,
              silu_in: bool = False, act_out: str | None = None) -> torch.Tensor:
    """bf16 linear y = act_out(bf16(act_in(a) w^T + bias)) on the matrix cores (wf_gemm_bf16)."""
    M, K = a.shape
    N = w.shape[0]
    if a.dtype != torch.bfloat16 or w.dtype != torch.bfloat16 or w.shape[1] != K or not w.is_contiguous():
        raise ValueError("gemm_bf16 takes bf16 a [M, K] and a contiguous bf16 w [N, K]")
    if a.stride(1) != 1 or a.stride(0) % 8 or a.data_ptr() % 16:
        a = a.contiguous()
    y = out if out is not None else torch.empty((M, N), dtype=torch.bfloat16, device=a.device)
    flags = (_lib.BF16_SILU_IN if silu_in else 0) | {None: 0, "silu": _lib.BF16_SILU_OUT,
                                                      "gelu": _lib.BF16_GELU_OUT}[act_out]
    _lib.call("wf_gemm_bf16", a.data_ptr(), M, K, a.stride(0), w.data_ptr(), N, _lib.ptr(bias), y.data_ptr(),
              y.stride(0), flags, _lib.stream_handle(a.device))
    return y


class QuantizedWanDiT:
    """The DiT of one chunk at one step: bf16 embeddings and head around a QuantizedWanStack."""

    def __init__(self, params: DiTParams, stack: QuantizedWanStack, schedule: FlowMatchSchedule | None = None):
        self.stack = stack
        self.device = stack.blocks[0].device
        dev = self.device
        self.dim = params.dim
        if self.dim != stack.blocks[0].dim:
            raise ValueError(f"DiT dim {self.dim} differs from the blocks' {stack.blocks[0].dim}")
        c = lambda t: t.to(dev).contiguous()
        self.patch_w = c(params.patch_w.reshape(self.dim, IN_DIM * 4))
        self.patch_b = c(params.patch_b)
        self.text1_w, self.text1_b = c(params.text1_w), c(params.text1_b)
        self.text2_w, self.text2_b = c(params.text2_w), c(params.text2_b)
        self.time1_w, self.time1_b = c(params.time1_w), c(params.time1_b)
        self.time2_w, self.time2_b = c(params.time2_w), c(params.time2_b)
        self.proj_w, self.proj_b = c(params.proj_w), c(params.proj_b)
        self.head_mod = c(params.head_mod)
        self.head_w, self.head_b = c(params.head_w), c(params.head_b)
        self.schedule = schedule if schedule is not None else FlowMatchSchedule()
        self._time: dict = {}
        self._ws: dict = {}

    # -- once per request
    def set_text(self, context: torch.Tensor) -> torch.Tensor:
        """Text embedding of the encoder output [L <= 512, 4096] (padded with zero rows to 512), and the
        cross-attention K/V of every layer from it.  Returns the embedded context [512, dim]."""
        if context.dim() != 2 or context.shape[1] != TEXT_DIM or context.shape[0] > TEXT_LEN:
            raise ValueError(f"context must be [L <= {TEXT_LEN}, {TEXT_DIM}], got {tuple(context.shape)}")
        ctx = torch.zeros((TEXT_LEN, TEXT_DIM), dtype=torch.bfloat16, device=self.device)
        ctx[:context.shape[0]] = context
        h = gemm_bf16(ctx, self.text1_w, self.text1_b, act_out="gelu")
        emb = gemm_bf16(h, self.text2_w, self.text2_b)
        self.stack.set_text(emb)
        return emb

    # -- per timestep (cached: the four DMD steps and the store pass's context noise recur every tick)
    def time_modulation(self, t: float, frames: int):
        """(e [F, dim], e0 [F, 6, dim]) bf16 of timestep t for each of the chunk's frames."""
        key = (float(t), frames)
        hit = self._time.get(key)
        if hit is None:
            s = sinusoidal_embedding(t, frames).to(torch.bfloat16).to(self.device)
            h = gemm_bf16(s, self.time1_w, self.time1_b, act_out="silu")
            e = gemm_bf16(h, self.time2_w, self.time2_b)
            e0 = gemm_bf16(e, self.proj_w, self.proj_b, silu_in=True).view(frames, 6, self.dim)
            if len(self._time) >= 64:
                self._time.clear()
            hit = self._time[key] = (e, e0)
        return hit

    def _workspace(self, T: int, slot: int = 0) -> dict:
        """Buffers of one pass over T tokens; concurrent passes use different slots."""
        ws = self._ws.get((T, slot))
        if ws is None:
            bf = dict(dtype=torch.bfloat16, device=self.device)
            ws = dict(patches=torch.empty((T, IN_DIM * 4), **bf), x=torch.empty((T, self.dim), **bf),
                      h=torch.empty((T, self.dim), **bf), flow=torch.empty((T, OUT_DIM * 4), **bf))
            self._ws[(T, slot)] = ws
        return ws

    @staticmethod
    def _check_latent(noisy: torch.Tensor) -> torch.Tensor:
        if noisy.dim() != 5 or noisy.shape[0] != 1 or noisy.shape[1] != IN_DIM or noisy.dtype != torch.bfloat16:
            raise ValueError(f"noisy must be bf16 [1, {IN_DIM}, F, H, W], got {tuple(noisy.shape)} {noisy.dtype}")
        return noisy.contiguous()

    def _embed(self, noisy: torch.Tensor, ws: dict) -> torch.Tensor:
        """Patch gather + patch embedding of a checked latent into ws["x"]."""
        _, C, Fr, H, W = noisy.shape
        _lib.call("wf_patchify_bf16", noisy.data_ptr(), 1, C, Fr, H, W, ws["patches"].data_ptr(),
                  _lib.stream_handle(self.device))
        return gemm_bf16(ws["patches"], self.patch_w, self.patch_b, out=ws["x"])

    def _head(self, x: torch.Tensor, e: torch.Tensor, noisy: torch.Tensor, t: float, ws: dict,
              x0: torch.Tensor) -> torch.Tensor:
        """Head (modulated LayerNorm, Linear(dim, 64)), unpatchify and x0 = xt - sigma * flow into x0."""
        _, C, Fr, H, W = noisy.shape
        T = x.shape[0]
        st = _lib.stream_handle(self.device)
        # head: LayerNorm + (shift, scale) = head modulation + e per frame, then Linear(dim, 64)
        es = self.head_mod[0].unsqueeze(0) + e.unsqueeze(1)          # [F, 2, dim] bf16
        _lib.call("wf_ln_modulate_quant", x.data_ptr(), T, self.dim, x.stride(0), EPS, None, None,
                  es[:, 0].data_ptr(), es[:, 1].data_ptr(), es.stride(0), T // Fr, ws["h"].data_ptr(),
                  ws["h"].stride(0), None, None, st)
        flow = gemm_bf16(ws["h"], self.head_w, self.head_b, out=ws["flow"])
        _lib.call("wf_unpatchify_flow_x0_bf16", flow.data_ptr(), noisy.data_ptr(), 1, C, Fr, H, W,
                  self.schedule.sigma_x0(t), x0.data_ptr(), st)
        return x0

    def _x0_buffer(self, noisy: torch.Tensor, x0_out: torch.Tensor | None) -> torch.Tensor:
        _, C, Fr, H, W = noisy.shape
        x0 = x0_out if x0_out is not None else torch.empty((1, Fr, C, H, W), dtype=torch.bfloat16, device=self.device)
        if tuple(x0.shape) != (1, Fr, C, H, W) or not x0.is_contiguous() or x0.dtype != torch.bfloat16:
            raise ValueError(f"x0_out must be contiguous bf16 [1, {Fr}, {C}, {H}, {W}]")
        return x0

    # -- one pass of a tick
    def run_pass(self, noisy: torch.Tensor, t: float, p: Pass, x0_out: torch.Tensor | None = None,
                 want_x0: bool = True) -> torch.Tensor | None:
        """The forward of noisy [1, 16, F, H, W] bf16 (B, C, T, H, W) at timestep t as pass p of the current tick;
        returns x0 [1, F, 16, H, W] bf16 (B, T, C, H, W), or None with ``want_x0=False`` (a store pass,
        whose x0 the wavefront drops: engine.py:383-389)."""
        noisy = self._check_latent(noisy)
        _, C, Fr, H, W = noisy.shape
        hp, wp = H // 2, W // 2
        ws = self._workspace(Fr * hp * wp)
        x = self._embed(noisy, ws)
        e, e0 = self.time_modulation(t, Fr)
        if not want_x0:
            # only the pages matter: the last layer stops after publishing its K/V
            self.stack.run_pass(x, e0, p, hp, wp, kv_only_last=True)
            return None
        self.stack.run_pass(x, e0, p, hp, wp)
        return self._head(x, e, noisy, t, ws, self._x0_buffer(noisy, x0_out))

    def tick(self, plan: TickPlan, inputs: dict, concurrent: bool = False) -> dict:
        """One wavefront tick on this GPU: ``inputs`` maps "store" (when the store rank is active) and each
        active denoise rank to (noisy [1, 16, F, H, W], timestep); the store pass runs first, then the ranks
        from the highest down (the order the reference's flag waits impose), one after another or
        (``concurrent``) as a layer wavefront on one stream per rank, with bit-identical results; returns
        {rank: x0} of the denoise passes (the store pass's x0 is dropped, as the reference drops it)."""
        ex = self.stack.exchange
        ex.begin_tick(plan)
        out = {}
        try:
            if plan.store_active:
                noisy, t = inputs["store"]
                self.run_pass(noisy, t, ex.store_pass(), want_x0=False)
            ranks = sorted(plan.act_ranks, reverse=True)
            if concurrent and len(ranks) > 1:
                out = self._denoise_wavefront(ranks, inputs, [ex.denoise_pass(r) for r in ranks])
            else:
                for r in ranks:
                    noisy, t = inputs[r]
                    out[r] = self.run_pass(noisy, t, ex.denoise_pass(r))
        except BaseException:
            ex.abort_tick()
            raise
        ex.end_tick()
        return out

    def _denoise_wavefront(self, ranks: list, inputs: dict, passes: list) -> dict:
        """The denoise passes of a tick as a layer wavefront (QuantizedWanStack.run_wavefront), each rank's
        patch embedding before and head after its layers on the rank's stream."""
        lat = [self._check_latent(inputs[r][0]) for r in ranks]
        ts = [inputs[r][1] for r in ranks]
        shapes = {tuple(n.shape) for n in lat}
        if len(shapes) != 1:
            raise ValueError(f"the ranks' latents differ in shape: {sorted(shapes)}")
        _, C, Fr, H, W = lat[0].shape
        hp, wp = H // 2, W // 2
        T = Fr * hp * wp
        wss = [self._workspace(T, slot=i) for i in range(len(ranks))]
        mods = [self.time_modulation(t, Fr) for t in ts]
        x0s = [self._x0_buffer(n, None) for n in lat]

        def pre(i):
            self._embed(lat[i], wss[i])

        def post(i):
            self._head(wss[i]["x"], mods[i][0], lat[i], ts[i], wss[i], x0s[i])

        self.stack.run_wavefront([(wss[i]["x"], mods[i][1], p) for i, p in enumerate(passes)],
                                 hp, wp, pre=pre, post=post)
        return dict(zip(ranks, x0s))

    def forward_chunk(self, noisy: torch.Tensor, t: float, start_frame: int | None = None, *,
                      chunk: int | None = None, store: bool = False):
        """One chunk alone as a tick of its own, called like ``WaveBackend.forward_chunk(noisy_chunk_bcthw,
        step_value, start_frame)`` (backend.py:456-490; ``start_frame`` a multiple of the chunk's frames, or
        the chunk index as ``chunk=``): a store pass (the chunk joins the clean lists; returns None) or a
        denoise pass of rank 0 (returns x0 [1, F, 16, H, W], B T C H W)."""
        ex = self.stack.exchange
        if (start_frame is None) == (chunk is None):
            raise ValueError("give exactly one of start_frame and chunk")
        if start_frame is not None:
            if start_frame < 0 or start_frame % ex.npb:
                raise ValueError(f"start_frame {start_frame} is not a chunk start (chunks of {ex.npb} frames)")
            chunk = start_frame // ex.npb
        Fr = noisy.shape[2]
        if store:
            self.tick(TickPlan(chunk + ex.rf_step, [], True, 0, 0), {"store": (noisy, t)})
            return None
        return self.tick(TickPlan(chunk, [0], False, chunk * ex.npb, Fr), {0: (noisy, t)})[0]
