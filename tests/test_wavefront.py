"""The wavefront loop's wiring on the CPU (WavefrontDenoiser.generate, engine.py:289-560), with the DiT and
the re-noising replaced by cheap stand-ins so every hand-off can be followed.

* each chunk's trajectory equals the chunk taken alone through the DMD steps: noise -> rank 0 at dsl[0]
  -> x0 -> re-noised to dsl[1] with seed stage 0 -> rank 1 ... -> rank rf-1's x0 -> the store pass at the
  context noise, which is the chunk's output; the stand-in x0 depends on the timestep and the stand-in
  re-noising on (timestep, chunk, stage), so a wrong step, chunk or seed changes the result;
* every tick's plan, ranks and chunks follow the reference's schedule (checked inside the stand-in tick);
* every stream starts on emptied clean lists (the exchange is reset), and bad noise shapes are refused.
"""

import types

import pytest
import torch

from waveforcing_amd import wavefront as wf
from waveforcing_amd.exchange import tick_plan
from waveforcing_amd.schedule import FlowMatchSchedule

NPB, H, W = 3, 4, 6


def _x0(latent_bcthw, t):
    """Stand-in forward: x0 [1, F, 16, H, W] (B, T, C, H, W) from a latent [1, 16, F, H, W] and its timestep."""
    return (latent_bcthw.float() * 0.5 + t / 1000.0).to(torch.bfloat16).permute(0, 2, 1, 3, 4).contiguous()


def _renoise(x0_bcthw, next_t, chunk, stage, schedule, out=None):
    return (x0_bcthw.float() + next_t / 100.0 + 10 * chunk + 100 * stage).to(torch.bfloat16)


class _FakeDiT:
    def __init__(self, rf_step):
        self.schedule = FlowMatchSchedule()
        ex = types.SimpleNamespace(rf_step=rf_step, npb=NPB, clean=[[], []], resets=0)

        def reset():
            ex.resets += 1
            ex.clean = [[], []]

        ex.reset = reset
        self.stack = types.SimpleNamespace(exchange=ex)
        self.seen = []

    def tick(self, plan, inputs, concurrent=False):
        rf = self.stack.exchange.rf_step
        assert sorted(k for k in inputs if k != "store") == sorted(plan.act_ranks)
        assert ("store" in inputs) == plan.store_active
        out = {}
        for r in plan.act_ranks:
            lat, t = inputs[r]
            assert lat.shape == (1, 16, NPB, H, W)
            self.seen.append((plan.tick, r, plan.tick - r, t))
            out[r] = _x0(lat, t)
        if plan.store_active:
            self.seen.append((plan.tick, "store", plan.tick - rf, inputs["store"][1]))
        return out


@pytest.mark.parametrize("rf_step,steps", [(4, (1000, 750, 500, 250)), (2, (1000, 500)), (1, (1000,))])
def test_generate_follows_each_chunks_trajectory(monkeypatch, rf_step, steps):
    monkeypatch.setattr(wf, "det_renoise", _renoise)
    dit = _FakeDiT(rf_step)
    den = wf.WavefrontDenoiser(dit, steps=steps, context_noise=0.0)
    n_chunks = 5
    noise = torch.randn((1, 16, NPB * n_chunks, H, W), generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    done = []
    out = den.generate(noise, on_chunk=lambda c, lat: done.append(c))
    dsl = dit.schedule.warp(steps)
    for c in range(n_chunks):
        lat = noise[:, :, c * NPB:(c + 1) * NPB]
        for r in range(rf_step):
            x0 = _x0(lat, dsl[r]).permute(0, 2, 1, 3, 4)
            lat = _renoise(x0, dsl[r + 1], c, r, None) if r < rf_step - 1 else x0
        assert torch.equal(out[:, :, c * NPB:(c + 1) * NPB], lat), f"chunk {c}"
    assert done == list(range(n_chunks))
    # the schedule: rank r at tick t holds chunk t - r at timestep dsl[r]; the store pass chunk t - rf_step
    want = []
    for t in range(n_chunks + rf_step):
        plan = tick_plan(t, rf_step, n_chunks, NPB)
        want += [(t, r, t - r, dsl[r]) for r in plan.act_ranks]
        if plan.store_active:
            want.append((t, "store", t - rf_step, 0.0))
    assert dit.seen == want


def test_generate_resets_the_exchange_and_refuses_bad_shapes(monkeypatch):
    monkeypatch.setattr(wf, "det_renoise", _renoise)
    dit = _FakeDiT(2)
    den = wf.WavefrontDenoiser(dit, steps=(1000, 500))
    with pytest.raises(ValueError, match="split into chunks"):
        den.generate(torch.zeros((1, 16, 4, H, W), dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="bf16"):
        den.generate(torch.zeros((1, 16, 3, H, W), dtype=torch.float32))
    assert dit.stack.exchange.resets == 0
    dit.stack.exchange.clean = [[object()], [object()]]
    den.generate(torch.zeros((1, 16, 3, H, W), dtype=torch.bfloat16))
    assert dit.stack.exchange.resets == 1
    with pytest.raises(ValueError, match="rf_step"):
        wf.WavefrontDenoiser(dit, steps=(1000, 750, 500))
