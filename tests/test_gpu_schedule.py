"""GPU parity of the re-noising kernel (wf_flow_add_noise_bf16) with the oracle.

Bit-exact against oracle.schedule.add_noise / det_renoise on the same inputs:
the 1.3B chunk latent [1, 16, 3, 60, 104] at each warped DMD sigma, a plane
that is not a multiple of 8 (one element per thread), batch 2, in-place
output, and _det_renoise's own draw (device generator seeded
1000 * chunk + stage, frame-major noise).
"""

import pytest
import torch

from oracle import schedule as osch
from waveforcing_amd import schedule as sch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _latent(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(torch.bfloat16)


@pytest.mark.parametrize("shape,frame_major", [
    ((1, 16, 3, 60, 104), True), ((1, 16, 3, 60, 104), False), ((2, 4, 3, 5, 7), True), ((2, 4, 3, 5, 7), False),
])
def test_add_noise_bit_exact(shape, frame_major):
    s = sch.FlowMatchSchedule()
    b, c, t, h, w = shape
    x0 = _latent(shape, 1)
    noise = _latent((b * t, c, h, w) if frame_major else shape, 2)
    for step in s.warp():
        sigma = s.sigma_at(step)
        got = sch.add_noise(x0.to(DEV), noise.to(DEV), sigma, noise_frame_major=frame_major).cpu()
        if frame_major:
            want = osch.det_renoise(x0, noise, torch.tensor(sigma))
        else:
            want = osch.add_noise(x0, noise, torch.tensor(sigma))
        assert torch.equal(got, want), (shape, frame_major, step)


def test_add_noise_in_place():
    x0 = _latent((1, 16, 3, 60, 104), 3).to(DEV)
    noise = _latent((1, 16, 3, 60, 104), 4).to(DEV)
    want = sch.add_noise(x0, noise, 0.625)
    sch.add_noise(x0, noise, 0.625, out=x0)
    assert torch.equal(x0, want)


def test_det_renoise_matches_oracle_with_the_reference_draw():
    s = sch.FlowMatchSchedule()
    x0 = _latent((1, 16, 3, 60, 104), 5).to(DEV)
    steps = s.warp()
    for stage in range(len(steps) - 1):
        chunk = 7
        got = sch.det_renoise(x0, steps[stage + 1], chunk, stage, s)
        noise = sch.renoise_noise(x0, chunk, stage)
        g = torch.Generator(device=DEV).manual_seed(1000 * chunk + stage)
        assert torch.equal(noise, torch.randn((3, 16, 60, 104), generator=g, device=DEV, dtype=torch.bfloat16))
        want = osch.det_renoise(x0.cpu(), noise.cpu(), torch.tensor(s.sigma_at(steps[stage + 1])))
        assert torch.equal(got.cpu(), want)


def test_add_noise_argument_errors():
    x0 = torch.zeros((1, 2, 3, 4, 4), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="noise must be"):
        sch.add_noise(x0, x0, 0.5, noise_frame_major=True)
    n = torch.zeros((3, 2, 4, 4), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="alias"):
        from waveforcing_amd import _lib
        _lib.call("wf_flow_add_noise_bf16", x0.data_ptr(), n.data_ptr(), 1, 2, 3, 16, 1, 0.5, n.data_ptr(),
                  _lib.stream_handle(DEV))
    torch.cuda.synchronize()
