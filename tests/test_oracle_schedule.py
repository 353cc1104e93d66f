"""Oracle of the flow-matching schedule and re-noising, pinned by closed forms.

* sigma(s) = shift * s / (1 + (shift - 1) * s) at s = 1 - k / 1000 (the
  linspace of set_timesteps with extra_one_step), evaluated in float64: the
  four warped DMD steps of the shipped step list (1000, 750, 500, 250) sit at
  sigma = 1, 15/16, 5/6 and 5/8 for shift 5;
* add_noise against (1 - sigma) x0 + sigma n in float64, to bf16 rounding;
* the frame-major noise order of _det_renoise, checked element by element on
  a tiny latent whose noise differs in every (frame, channel) position (a
  transposed read fails it).
The host-side table of waveforcing_amd.schedule must equal the oracle's.
"""

import pytest
import torch

from oracle import schedule as osch
from waveforcing_amd import schedule as sch


def test_sigmas_closed_form():
    sig, ts = osch.flow_sigmas(shift=5.0)
    assert sig.dtype == torch.float32 and sig.shape == (1000,)
    s = 1 - torch.arange(1000, dtype=torch.float64) / 1000
    want = 5 * s / (1 + 4 * s)
    assert float((sig.double() - want).abs().max()) <= 2e-7
    assert float(sig[0]) == 1.0 and bool((sig[1:] < sig[:-1]).all())
    assert torch.equal(ts, sig * 1000)


def test_warped_dmd_steps():
    sig, ts = osch.flow_sigmas(shift=5.0)
    got = osch.warp_steps(ts, (1000, 750, 500, 250)).double()
    want = torch.tensor([1000.0, 937.5, 2500.0 / 3, 625.0], dtype=torch.float64)
    assert float((got - want).abs().max()) <= 1e-4
    assert float(osch.warp_steps(ts, (0,))) == 0.0          # the appended 0
    for t, s in zip(got.tolist(), (1.0, 15 / 16, 5 / 6, 5 / 8)):
        assert abs(float(osch.sigma_at(sig, ts, t)) - s) <= 1e-6


def test_sigma_at_nearest_and_first_on_tie():
    sig, ts = osch.flow_sigmas(shift=5.0)
    assert float(osch.sigma_at(sig, ts, 0.0)) == float(sig[-1])      # below the table: the last entry
    mid = (float(ts[10]) + float(ts[11])) / 2
    i = int(torch.argmin((ts - torch.tensor(mid, dtype=torch.float32)).abs()))
    assert float(osch.sigma_at(sig, ts, mid)) == float(sig[i])


def test_add_noise_closed_form():
    g = torch.Generator().manual_seed(0)
    x0 = torch.randn((2, 3, 4, 5), generator=g).to(torch.bfloat16)
    n = torch.randn((2, 3, 4, 5), generator=g).to(torch.bfloat16)
    for sigma in (1.0, 15 / 16, 0.625, 0.0):
        s = torch.tensor(sigma, dtype=torch.float32)
        got = osch.add_noise(x0, n, s).double()
        sd = float(s)
        want = (1 - sd) * x0.double() + sd * n.double()
        assert bool(((got - want).abs() <= want.abs() * 2 ** -8 + 1e-6).all())
    assert torch.equal(osch.add_noise(x0, n, torch.tensor(1.0)), n)
    assert torch.equal(osch.add_noise(x0, n, torch.tensor(0.0)), x0)


def test_det_renoise_reads_noise_frame_major():
    B, C, T, H, W = 1, 3, 2, 2, 2
    x0 = torch.zeros((B, C, T, H, W), dtype=torch.bfloat16)
    noise = torch.empty((B * T, C, H, W), dtype=torch.bfloat16)
    for t in range(T):
        for c in range(C):
            noise[t, c] = 10 * t + c + 1                    # distinct per (frame, channel)
    out = osch.det_renoise(x0, noise, torch.tensor(1.0))
    for c in range(C):
        for t in range(T):
            assert bool((out[0, c, t] == 10 * t + c + 1).all())


@pytest.mark.parametrize("shift", [5.0, 8.0, 3.0])
def test_host_schedule_equals_oracle(shift):
    s = sch.FlowMatchSchedule(shift=shift)
    sig, ts = osch.flow_sigmas(shift=shift)
    assert torch.equal(s.sigmas, sig) and torch.equal(s.timesteps, ts)
    assert s.warp() == [float(x) for x in osch.warp_steps(ts, sch.DMD_STEPS)]
    for t in s.warp() + [0.0, 123.4, 999.9]:
        assert s.sigma_at(t) == float(osch.sigma_at(sig, ts, t))
    with pytest.raises(ValueError, match="outside"):
        s.warp((1001,))
