"""The wavefront denoising loop on one GPU: a stream of chunks from noise to clean latents.

Restates WaveDenoiser's tick loop (wave_rt/denoiser/engine.py:289-560) with
every rank on this GPU.  At tick t (``num_chunks + rf_step`` ticks in all,
engine.py:53):

* denoise rank r holds chunk c = t - r at DMD step r (timestep
  ``dsl[r]``, the warped step list): rank 0 takes chunk c of the noise
  (engine.py:318-323); rank r > 0 takes the x0 that rank r - 1 produced at the
  previous tick, re-noised to ``dsl[r]`` with the seed ``1000 c + (r - 1)``
  (``_det_renoise``, engine.py:221-235,530-540);
* the store rank holds chunk t - rf_step: the x0 of the last denoise rank from
  the previous tick, passed on without re-noising (engine.py:536-540), run at
  the context noise timestep so that its K/V join every layer's clean list
  (engine.py:383-389); that latent is the chunk's final output
  (engine.py:390).

The tick itself is QuantizedWanDiT.tick (one GPU: the store pass, then the
denoise ranks, optionally as a layer wavefront on one stream per rank); the
"latent migration" between ranks is the hand-off of tensors on this GPU.
"""

from __future__ import annotations

import torch

from .dit import IN_DIM, QuantizedWanDiT
from .exchange import tick_plan
from .schedule import DMD_STEPS, det_renoise


class WavefrontDenoiser:
    """WaveDenoiser's loop over one GPU's QuantizedWanDiT (which holds the paged exchange)."""

    def __init__(self, dit: QuantizedWanDiT, steps=DMD_STEPS, context_noise: float = 0.0) -> None:
        self.dit = dit
        ex = dit.stack.exchange
        self.rf_step = ex.rf_step
        self.npb = ex.npb
        self.dsl = dit.schedule.warp(steps)
        if len(self.dsl) != self.rf_step:
            # one DMD step per denoise rank (config.py:84-88)
            raise ValueError(f"{len(self.dsl)} denoising steps for rf_step {self.rf_step}")
        self.context_noise = float(context_noise)

    def generate(self, noise: torch.Tensor, concurrent: bool = False, on_chunk=None) -> torch.Tensor:
        """Denoise ``noise`` [1, 16, F, H, W] bf16 (F a multiple of the chunk's frames) chunk by chunk through
        the wavefront; returns the clean latents [1, 16, F, H, W] (each chunk's store-pass input).
        ``on_chunk(c, latent)``, if given, is called as each chunk completes (the reference's output queue,
        engine.py:391-403).  The stream starts at chunk 0 on emptied clean lists (PagedExchange.reset,
        engine.py:294)."""
        if noise.dim() != 5 or noise.shape[0] != 1 or noise.shape[1] != IN_DIM or noise.dtype != torch.bfloat16:
            raise ValueError(f"noise must be bf16 [1, {IN_DIM}, F, H, W], got {tuple(noise.shape)} {noise.dtype}")
        npb, rf = self.npb, self.rf_step
        if noise.shape[2] % npb:
            raise ValueError(f"{noise.shape[2]} latent frames do not split into chunks of {npb}")
        self.dit.stack.exchange.reset()
        num_chunks = noise.shape[2] // npb
        out = torch.empty_like(noise)
        handoff: dict = {}       # rank (or "store") -> latent [1, 16, npb, H, W] it takes at the next tick
        for t in range(num_chunks + rf):
            plan = tick_plan(t, rf, num_chunks, npb)
            inputs = {}
            for r in plan.act_ranks:
                c = t - r
                lat = noise[:, :, c * npb:(c + 1) * npb].contiguous() if r == 0 else handoff.pop(r)
                inputs[r] = (lat, self.dsl[r])
            if plan.store_active:
                inputs["store"] = (handoff.pop("store"), self.context_noise)
            x0s = self.dit.tick(plan, inputs, concurrent=concurrent)
            if plan.store_active:
                c = t - rf
                out[:, :, c * npb:(c + 1) * npb] = inputs["store"][0]
                if on_chunk is not None:
                    on_chunk(c, inputs["store"][0])
            for r, x0 in x0s.items():
                c = t - r
                x0_bcthw = x0.permute(0, 2, 1, 3, 4).contiguous()
                if r < rf - 1:
                    handoff[r + 1] = det_renoise(x0_bcthw, self.dsl[r + 1], c, r, self.dit.schedule)
                else:
                    handoff["store"] = x0_bcthw
        return out
