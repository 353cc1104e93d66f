"""Flow-matching schedule and deterministic re-noising oracle (torch CPU).

Test infrastructure only: what waveforcing_amd.schedule is tested against.

* Sigma / timestep table of FlowMatchScheduler.set_timesteps
  (naive_rt/rolling_forcing/utils/scheduler.py:108-136) with the generator's
  arguments (wan_wrapper.py:136-139: shift = timestep_shift, sigma_min = 0,
  extra_one_step = True, set_timesteps(1000, training=True)), in float32 as
  torch evaluates it there.
* The warped DMD step list (rolling_forcing_inference.py:24-28): the
  timesteps with a trailing 0, indexed at 1000 - step.
* add_noise (scheduler.py:159-176): sigma at the nearest timestep, then
  ``(1 - sigma) * x0 + sigma * noise`` in float32, cast to the noise dtype.
* _det_renoise (wave_rt/denoiser/engine.py:221-235): x0 [B, C, T, H, W] is
  viewed frame-major, noise is drawn in that [B*T, C, H, W] order, and the
  result is permuted back to [B, C, T, H, W].
"""

from __future__ import annotations

import torch


def flow_sigmas(num_steps: int = 1000, shift: float = 5.0, sigma_min: float = 0.0, sigma_max: float = 1.0,
                extra_one_step: bool = True):
    """(sigmas, timesteps) float32 [num_steps] (scheduler.py:119-134, no inversion or reversal)."""
    sigma_start = sigma_min + (sigma_max - sigma_min) * 1.0
    if extra_one_step:
        s = torch.linspace(sigma_start, sigma_min, num_steps + 1)[:-1]
    else:
        s = torch.linspace(sigma_start, sigma_min, num_steps)
    s = shift * s / (1 + (shift - 1) * s)
    return s, s * 1000


def warp_steps(timesteps: torch.Tensor, steps) -> torch.Tensor:
    """Warped denoising step list (rolling_forcing_inference.py:26-28)."""
    t = torch.cat((timesteps.cpu(), torch.tensor([0], dtype=torch.float32)))
    return t[1000 - torch.tensor(list(steps), dtype=torch.long)]


def sigma_at(sigmas: torch.Tensor, timesteps: torch.Tensor, t: float) -> torch.Tensor:
    """sigma of the timestep nearest to t (scheduler.py:171-173), float32 scalar tensor."""
    tt = float(t) * torch.ones([1], dtype=torch.long)
    idx = torch.argmin((timesteps.unsqueeze(0) - tt.unsqueeze(1)).abs(), dim=1)
    return sigmas[idx].reshape(())


def add_noise(x0: torch.Tensor, noise: torch.Tensor, sigma: torch.Tensor) -> torch.Tensor:
    """(1 - sigma) * x0 + sigma * noise in float32, cast to noise's dtype (scheduler.py:174-175)."""
    s = sigma.reshape(1).float()
    return ((1 - s) * x0 + s * noise).type_as(noise)


def det_renoise(x0_bcthw: torch.Tensor, noise_btchw: torch.Tensor, sigma: torch.Tensor) -> torch.Tensor:
    """engine.py:221-235 given the drawn noise [B*T, C, H, W] (frame-major)."""
    b, c, t, h, w = x0_bcthw.shape
    flat = x0_bcthw.permute(0, 2, 1, 3, 4).flatten(0, 1)
    out = add_noise(flat, noise_btchw.reshape(b * t, c, h, w), sigma).unflatten(0, (b, t))
    return out.permute(0, 2, 1, 3, 4).contiguous()
