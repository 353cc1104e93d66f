"""Flow-matching DMD schedule and the deterministic re-noising between steps.

Between two denoising steps of a chunk, the x0 prediction of step ``stage``
is re-noised to the next step's timestep before it moves on (the latent
migration of WaveDenoiser, wave_rt/denoiser/engine.py:525-555, whose payload
is ``_det_renoise``, :221-235).  On one GPU there is nothing to migrate: the
re-noised latent is the next step's input on the same device.

* :class:`FlowMatchSchedule` holds the sigma / timestep table of
  FlowMatchScheduler.set_timesteps (naive_rt/rolling_forcing/utils/
  scheduler.py:108-136) built as the generator builds it (wan_wrapper.py:
  136-139: ``shift = timestep_shift``, ``sigma_min = 0``,
  ``extra_one_step = True``, ``set_timesteps(1000, training=True)``), in
  float32, and the warped DMD step list (rolling_forcing_inference.py:26-28).
* :func:`add_noise` is ``(1 - sigma) * x0 + sigma * noise`` in float32, cast
  to bf16 (scheduler.py:159-176), as one HIP kernel (wf_flow_add_noise_bf16).
* :func:`det_renoise` draws the noise as _det_renoise does -- a generator on
  the latent's device seeded ``1000 * chunk + stage``, ``randn`` in the
  frame-major [B*T, C, H, W] order of the latent's permuted view -- and lets
  the kernel read it in that order, without the permuted copies.  The draw is
  torch's device generator, so it equals the reference's draw on the same
  kind of device.
"""

from __future__ import annotations

import torch

from . import _lib

DMD_STEPS = (1000, 750, 500, 250)   # denoising_step_list (wave_rt/config.py:30)


class FlowMatchSchedule:
    """Sigma / timestep table of the rolling-forcing generator's FlowMatchScheduler."""

    def __init__(self, shift: float = 5.0, num_steps: int = 1000, sigma_min: float = 0.0, sigma_max: float = 1.0,
                 extra_one_step: bool = True) -> None:
        # set_timesteps(num_steps, denoising_strength=1.0): the same float32 torch operations
        start = sigma_min + (sigma_max - sigma_min) * 1.0
        n = num_steps + 1 if extra_one_step else num_steps
        s = torch.linspace(start, sigma_min, n)
        if extra_one_step:
            s = s[:-1]
        self.shift = shift
        self.sigmas = shift * s / (1 + (shift - 1) * s)
        self.timesteps = self.sigmas * 1000       # num_train_timesteps (the class default)

    def warp(self, steps=DMD_STEPS) -> list[float]:
        """Warped denoising step list: the timesteps with a trailing 0, at 1000 - step."""
        t = torch.cat((self.timesteps, torch.tensor([0], dtype=torch.float32)))
        idx = torch.tensor([1000 - int(x) for x in steps], dtype=torch.long)
        if bool((idx < 0).any()) or bool((idx >= t.numel()).any()):
            raise ValueError(f"denoising steps {list(steps)} fall outside the 1000-step table")
        return [float(x) for x in t[idx]]

    def sigma_x0(self, t: float) -> float:
        """sigma of the timestep nearest to t as the flow -> x0 conversion picks it: in float64 over the
        float32 table (wan_wrapper.py:182-190)."""
        ts = self.timesteps.double()
        idx = int(torch.argmin((ts - float(t)).abs()))
        return float(self.sigmas.double()[idx])

    def sigma_at(self, t: float) -> float:
        """sigma of the timestep nearest to t (the first on a tie), as add_noise picks it."""
        tt = float(t) * torch.ones([1], dtype=torch.long)
        idx = int(torch.argmin((self.timesteps.unsqueeze(0) - tt.unsqueeze(1)).abs(), dim=1))
        return float(self.sigmas[idx])


def _check(x: torch.Tensor, name: str) -> None:
    if x.dtype != torch.bfloat16 or not x.is_contiguous() or x.device.type != "cuda":
        raise ValueError(f"{name} must be a contiguous bf16 CUDA tensor, got {x.dtype} on {x.device}")


def add_noise(x0_bcthw: torch.Tensor, noise: torch.Tensor, sigma: float, noise_frame_major: bool = False,
              out: torch.Tensor | None = None) -> torch.Tensor:
    """bf16((1 - sigma) * x0 + sigma * noise) of a latent x0 [B, C, T, H, W].

    noise is [B, C, T, H, W], or [B*T, C, H, W] frame-major with
    ``noise_frame_major``; out (default new) may be x0 itself.
    """
    if x0_bcthw.dim() != 5:
        raise ValueError(f"x0 must be [B, C, T, H, W], got {tuple(x0_bcthw.shape)}")
    b, c, t, h, w = x0_bcthw.shape
    want = (b * t, c, h, w) if noise_frame_major else (b, c, t, h, w)
    if tuple(noise.shape) != want:
        raise ValueError(f"noise must be {want}, got {tuple(noise.shape)}")
    out = torch.empty_like(x0_bcthw) if out is None else out
    if out.shape != x0_bcthw.shape:
        raise ValueError(f"out {tuple(out.shape)} differs from x0 {tuple(x0_bcthw.shape)}")
    for name, tns in (("x0", x0_bcthw), ("noise", noise), ("out", out)):
        _check(tns, name)
    _lib.call("wf_flow_add_noise_bf16", x0_bcthw.data_ptr(), noise.data_ptr(), b, c, t, h * w,
              1 if noise_frame_major else 0, float(sigma), out.data_ptr(), _lib.stream_handle(x0_bcthw.device))
    return out


def renoise_noise(x0_bcthw: torch.Tensor, chunk: int, stage: int) -> torch.Tensor:
    """The noise _det_renoise draws for (chunk, stage): frame-major [B*T, C, H, W] in x0's dtype."""
    b, c, t, h, w = x0_bcthw.shape
    g = torch.Generator(device=x0_bcthw.device).manual_seed(1000 * chunk + stage)
    return torch.randn((b * t, c, h, w), generator=g, device=x0_bcthw.device, dtype=x0_bcthw.dtype)


def det_renoise(x0_bcthw: torch.Tensor, next_t: float, chunk: int, stage: int, schedule: FlowMatchSchedule,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """_det_renoise (engine.py:221-235): x0 [B, C, T, H, W] bf16 re-noised to timestep next_t."""
    noise = renoise_noise(x0_bcthw, chunk, stage)
    return add_noise(x0_bcthw, noise, schedule.sigma_at(next_t), noise_frame_major=True, out=out)
