"""GPU parity of the DiT layers around the blocks against the CPU oracle (oracle/dit.py).

* wf_gemm_bf16 at the shapes of the patch embedding, text and time
  embeddings, time projection and head: within one bf16 ulp of the oracle's
  fp32-accumulated linear (a different summation order may move the single
  rounding by one ulp) in all but a few elements; with SiLU / GELU(tanh), whose
  exponential differs from the CPU's, relative L2 <= 1e-3;
* patch gather: bit-exact;
* unpatchify + flow -> x0: bit-exact (float64 arithmetic, float32 route to bf16);
* the time and text embeddings of QuantizedWanDiT with the one-hot probes of
  tests/embed_probes.py: within one bf16 ulp of the float64 definitions of
  their SiLU / GELU(tanh) activations, the text padding rows equal to the
  second bias bit for bit;
* one chunk's whole forward (QuantizedWanDiT.forward_chunk: patch embedding,
  time embedding, 2 blocks over the paged exchange, head, x0) against the
  oracle chained over the same parameters, at a small width and at the 1.3B
  width on a 4680-token chunk: relative L2 <= 1e-2 (the block bar).
"""

import pytest
import torch

import embed_probes as ep
from oracle import block as ob
from oracle import dit as od
from oracle import kv as okv
from waveforcing_amd import _lib
from waveforcing_amd.block import QuantizedWanBlock, random_block_params
from waveforcing_amd.dit import QuantizedWanDiT, gemm_bf16, random_dit_params
from waveforcing_amd.exchange import PagedExchange, tick_plan
from waveforcing_amd.schedule import FlowMatchSchedule
from waveforcing_amd.stack import QuantizedWanStack

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
BF16 = torch.bfloat16


def _ulp(x):
    return torch.pow(2.0, torch.floor(torch.log2(x.abs().clamp(min=2.0 ** -100))) - 7)


@pytest.mark.parametrize("M,K,N,silu_in,act", [
    (4680, 64, 1536, False, None),      # patch embedding
    (512, 4096, 1536, False, "gelu"),   # text embedding, first linear
    (512, 1536, 1536, False, None),     # text embedding, second linear
    (3, 256, 1536, False, "silu"),      # time embedding, first linear
    (3, 1536, 9216, True, None),        # time projection (SiLU first)
    (4680, 1536, 64, False, None),      # head
    (4680, 5120, 64, False, None),      # 14B head
    (37, 40, 12, False, None), (1, 8, 4, True, "silu"),
])
def test_gemm_bf16_matches_oracle_linear(M, K, N, silu_in, act):
    g = torch.Generator().manual_seed(M + K + N)
    a = torch.randn((M, K), generator=g).to(BF16)
    w = (torch.randn((N, K), generator=g) * K ** -0.5).to(BF16)
    b = (torch.randn((N,), generator=g) * 0.1).to(BF16)
    got = gemm_bf16(a.to(DEV), w.to(DEV), b.to(DEV), silu_in=silu_in, act_out=act).cpu().float()
    want = od.linear(a, w, b, act_out=act, silu_in=silu_in).float()
    rel = ((got - want).norm() / want.norm()).item()
    print(f"rel L2 {rel:.2e}")
    if act is None and not silu_in:
        assert ((got - want).abs() <= _ulp(want) + 1e-6).all()
        assert (got == want).double().mean() > 0.98
    assert rel <= 1e-3


def test_patchify_exact():
    lat = torch.randn((1, 16, 3, 60, 104), generator=torch.Generator().manual_seed(1)).to(BF16)
    out = torch.empty((3 * 30 * 52, 64), dtype=BF16, device=DEV)
    lat_d = lat.to(DEV)   # held: a temporary's memory could be handed to the next allocation before the launch
    _lib.call("wf_patchify_bf16", lat_d.data_ptr(), 1, 16, 3, 60, 104, out.data_ptr(), _lib.stream_handle(DEV))
    assert torch.equal(out.cpu(), od.patchify(lat[0]))


@pytest.mark.parametrize("sigma", [0.0, 15 / 16, 0.8333333333333334, 0.625, 1.0])
def test_unpatchify_flow_x0_exact(sigma):
    g = torch.Generator().manual_seed(2)
    head = torch.randn((3 * 30 * 52, 64), generator=g).to(BF16)
    xt = torch.randn((1, 16, 3, 60, 104), generator=g).to(BF16)
    x0 = torch.empty((1, 3, 16, 60, 104), dtype=BF16, device=DEV)
    head_d, xt_d = head.to(DEV), xt.to(DEV)
    _lib.call("wf_unpatchify_flow_x0_bf16", head_d.data_ptr(), xt_d.data_ptr(), 1, 16, 3, 60, 104,
              float(sigma), x0.data_ptr(), _lib.stream_handle(DEV))
    want = od.flow_to_x0(od.unpatchify(head, (3, 30, 52)), xt[0], sigma).permute(1, 0, 2, 3)
    assert torch.equal(x0.cpu()[0], want)


def _probe_dit(dparams, dim=256, heads=2, ffn=512):
    blocks = [QuantizedWanBlock(random_block_params(dim, ffn, seed=1), heads, DEV)]
    stack = QuantizedWanStack(blocks, PagedExchange(1, heads, 64, 3, 21, rf_step=4, device=DEV))
    return QuantizedWanDiT(dparams, stack)


@pytest.mark.parametrize("t", [1000.0, 937.5, 625.0, 3.0])
def test_time_embedding_probe_closed_form(t):
    p, picks = ep.time_probe(random_dit_params(256, seed=9))
    e, e0 = _probe_dit(p).time_modulation(t, 3)
    want_e, want_e0 = ep.time_closed_form(t, 3, picks)
    print(f"e exact {(e.cpu() == want_e).double().mean().item():.4f}, "
          f"e0 exact {(e0.cpu() == want_e0).double().mean().item():.4f}")
    assert ep.within_one_ulp(e.cpu(), want_e) and ep.within_one_ulp(e0.cpu(), want_e0)


def test_text_embedding_probe_closed_form():
    p, ctx, picks = ep.text_probe(random_dit_params(256, seed=10))
    got = _probe_dit(p).set_text(ctx.to(DEV)).cpu()
    want = ep.text_closed_form(ctx, p.text2_b, picks)
    print(f"exact {(got == want).double().mean().item():.4f}")
    assert ep.within_one_ulp(got, want)
    assert torch.equal(got[ctx.shape[0]:], p.text2_b.expand(512 - ctx.shape[0], 256))


def _dit_case(dim, heads, ffn, layers, H, W, seed):
    bparams = [random_block_params(dim, ffn, seed=seed + i) for i in range(layers)]
    dparams = random_dit_params(dim, seed=seed + 100)
    g = torch.Generator().manual_seed(seed + 200)
    noisy = torch.randn((1, 16, 3, H, W), generator=g).to(BF16)
    ctx = (torch.randn((300, 4096), generator=g) * 0.5).to(BF16)
    return bparams, dparams, noisy, ctx


@pytest.mark.parametrize("dim,heads,ffn,H,W", [(256, 2, 512, 16, 16), (1536, 12, 8960, 60, 104)])
def test_dit_forward_chunk_matches_oracle(dim, heads, ffn, H, W):
    layers, t = 2, 937.5
    bparams, dparams, noisy, ctx = _dit_case(dim, heads, ffn, layers, H, W, seed=11)
    hp, wp = H // 2, W // 2
    page = hp * wp
    T = 3 * page
    # GPU: a fresh exchange (no clean chunks): the first denoise pass of chunk 0 attends to itself
    blocks = [QuantizedWanBlock(p, heads, DEV) for p in bparams]
    stack = QuantizedWanStack(blocks, PagedExchange(layers, heads, page, 3, 21, rf_step=4, device=DEV))
    dit = QuantizedWanDiT(dparams, stack)
    emb = dit.set_text(ctx.to(DEV))
    x0 = dit.forward_chunk(noisy.to(DEV), t, chunk=0).cpu()[0]
    # oracle
    oemb = od.text_embed(dparams, ctx)
    emb_rel = ((emb.cpu().float() - oemb.float()).norm() / oemb.float().norm()).item()
    tkv = [ob.text_kv(p, oemb, heads) for p in bparams]

    def stack_fn(x, e0):
        for L, p in enumerate(bparams):
            pk, pv = okv.new_pool(3, page, heads, 128), okv.new_pool(3, page, heads, 128)
            x = ob.block_forward(p, x, e0, (3, hp, wp), 0, pk, pv, [0, 1, 2], [0, 1, 2], T, page, *tkv[L], heads)
        return x

    sched = FlowMatchSchedule()
    sig, ts = sched.sigmas, sched.timesteps
    want = od.dit_forward(dparams, stack_fn, noisy[0], t, od.sigma_x0(sig, ts, t))
    rel = ((x0.float() - want.float()).norm() / want.float().norm()).item()
    # the flow part alone (x0 - xt = -sigma * flow) carries the blocks' differences
    xt = noisy[0].permute(1, 0, 2, 3).float()
    frel = (((x0.float() - xt) - (want.float() - xt)).norm() / (want.float() - xt).norm()).item()
    print(f"text embedding rel L2 {emb_rel:.2e}; x0 rel L2 {rel:.2e}; flow part rel L2 {frel:.2e}")
    assert emb_rel <= 1e-2
    assert frel <= 1e-2


def test_dit_concurrent_tick_is_bit_identical():
    """QuantizedWanDiT.tick(concurrent=True) -- the denoise ranks' patch embedding, layers and head on one
    stream per rank as a layer wavefront -- returns the same x0, bit for bit, as the sequential tick, over
    the ticks of a short stream at rf_step 4."""
    dim, heads, ffn, layers, H, W = 256, 2, 512, 2, 16, 16
    bparams, dparams, _, ctx = _dit_case(dim, heads, ffn, layers, H, W, seed=31)
    page = (H // 2) * (W // 2)

    def make():
        blocks = [QuantizedWanBlock(p, heads, DEV) for p in bparams]
        dit = QuantizedWanDiT(dparams, QuantizedWanStack(blocks, PagedExchange(layers, heads, page, 3, 21, rf_step=4,
                                                                                device=DEV)))
        dit.set_text(ctx.to(DEV))
        return dit

    seq, con = make(), make()
    steps = seq.schedule.warp()
    n_chunks = 6
    for t in range(n_chunks + 4):
        plan = tick_plan(t, 4, n_chunks, 3)
        ins = {}
        if plan.store_active:
            ins["store"] = (torch.randn((1, 16, 3, H, W), generator=torch.Generator().manual_seed(t)).to(BF16), 0.0)
        for r in plan.act_ranks:
            g = torch.Generator().manual_seed(100 * t + r)
            ins[r] = (torch.randn((1, 16, 3, H, W), generator=g).to(BF16), steps[r])
        dev_ins = {k: (x.to(DEV), tt) for k, (x, tt) in ins.items()}
        a = seq.tick(plan, dev_ins)
        b = con.tick(tick_plan(t, 4, n_chunks, 3), dev_ins, concurrent=True)
        torch.cuda.synchronize()
        assert sorted(a) == sorted(b) == sorted(plan.act_ranks)
        for r in a:
            assert torch.equal(a[r], b[r]), f"tick {t} rank {r}"


def test_wavefront_generate_sequential_and_concurrent_agree():
    """WavefrontDenoiser.generate over 5 chunks at rf_step 4 (the loop of engine.py:289-560 on one GPU):
    the sequential and the concurrent tick give the same clean latents, bit for bit, and so does a second
    stream on the same DiT (the exchange reset between streams); chunk 0 -- which has
    no older chunk to attend to -- equals its trajectory replayed alone on a fresh DiT (rank 0's pass at each
    DMD step through forward_chunk, re-noised between steps with seed 1000 * 0 + stage)."""
    from waveforcing_amd.schedule import det_renoise
    from waveforcing_amd.wavefront import WavefrontDenoiser

    dim, heads, ffn, layers, H, W = 256, 2, 512, 2, 16, 16
    bparams, dparams, _, ctx = _dit_case(dim, heads, ffn, layers, H, W, seed=41)
    page = (H // 2) * (W // 2)

    def make():
        blocks = [QuantizedWanBlock(p, heads, DEV) for p in bparams]
        dit = QuantizedWanDiT(dparams, QuantizedWanStack(blocks, PagedExchange(layers, heads, page, 3, 21, rf_step=4,
                                                                                device=DEV)))
        dit.set_text(ctx.to(DEV))
        return dit

    n_chunks = 5
    noise = torch.randn((1, 16, 3 * n_chunks, H, W), generator=torch.Generator().manual_seed(42)).to(BF16).to(DEV)
    done = []
    seq_dit = make()
    seq = WavefrontDenoiser(seq_dit).generate(noise, on_chunk=lambda c, lat: done.append(c))
    con = WavefrontDenoiser(make()).generate(noise, concurrent=True)
    torch.cuda.synchronize()
    assert done == list(range(n_chunks))
    assert torch.isfinite(seq.float()).all()
    assert torch.equal(seq, con)
    # every chunk's store pass added one clean page per layer
    assert all(len(c) == n_chunks for c in seq_dit.stack.exchange.clean)
    # a second stream on the same DiT starts from emptied clean lists and repeats the first exactly
    again = WavefrontDenoiser(seq_dit).generate(noise, concurrent=True)
    torch.cuda.synchronize()
    assert torch.equal(again, seq)

    alone = make()
    dsl = alone.schedule.warp()
    lat = noise[:, :, 0:3].contiguous()
    for r in range(4):
        x0 = alone.forward_chunk(lat, dsl[r], chunk=0).permute(0, 2, 1, 3, 4).contiguous()
        lat = det_renoise(x0, dsl[r + 1], 0, r, alone.schedule) if r < 3 else x0
    torch.cuda.synchronize()
    assert torch.equal(seq[:, :, 0:3], lat)


def test_store_pass_stops_after_the_last_layers_kv():
    """A store pass whose output is dropped (run_pass with want_x0=False) runs its last layer only up to the
    K/V pack: over three stored chunks the pool's codes and scales and the anchor's un-rotated K equal those
    the whole pass (through the last layer's FFN and the head) leaves, bit for bit, and so does the x0 of a
    denoise pass over that context."""
    from waveforcing_amd.exchange import TickPlan

    dim, heads, ffn, layers, H, W = 256, 2, 512, 2, 16, 16
    bparams, dparams, noisy, ctx = _dit_case(dim, heads, ffn, layers, H, W, seed=51)
    page = (H // 2) * (W // 2)

    def make():
        blocks = [QuantizedWanBlock(p, heads, DEV) for p in bparams]
        dit = QuantizedWanDiT(dparams, QuantizedWanStack(blocks, PagedExchange(layers, heads, page, 3, 21, rf_step=4,
                                                                                device=DEV)))
        dit.set_text(ctx.to(DEV))
        return dit

    short, full = make(), make()
    g = torch.Generator().manual_seed(52)
    for c in range(3):
        lat = torch.randn((1, 16, 3, H, W), generator=g).to(BF16).to(DEV)
        short.forward_chunk(lat, 0.0, chunk=c, store=True)
        ex = full.stack.exchange
        ex.begin_tick(TickPlan(c + 4, [], True, 0, 0))
        full.run_pass(lat, 0.0, ex.store_pass(), want_x0=True)
        ex.end_tick()
    torch.cuda.synchronize()
    a, b = short.stack.exchange, full.stack.exchange
    for name in ("k_codes", "v_codes", "k_scales", "v_scales"):
        assert torch.equal(getattr(a.pool, name), getattr(b.pool, name)), name
    assert torch.equal(a.anchor_ku, b.anchor_ku)
    x0a = short.forward_chunk(noisy.to(DEV), 937.5, chunk=3)
    x0b = full.forward_chunk(noisy.to(DEV), 937.5, 9)     # the reference's call: start_frame = 3 chunks x 3
    torch.cuda.synchronize()
    assert torch.equal(x0a, x0b)
    with pytest.raises(ValueError, match="chunk start"):
        full.forward_chunk(noisy.to(DEV), 937.5, 4)
    with pytest.raises(ValueError, match="exactly one"):
        full.forward_chunk(noisy.to(DEV), 937.5, 9, chunk=3)


def test_wavefront_stream_passes_match_the_oracle():
    """Every denoise pass of a 4-chunk stream at rf_step 2 (WavefrontDenoiser.generate: noise in, re-noised
    hand-offs between the two DMD steps, store passes at the context noise) against the oracle DiT forward
    fed the latent and timestep the pass was given, over the reference's context for that pass (the list
    model of exchange_model: anchor re-RoPEd to the pass's start, working chunks, the live stored chunk,
    the in-flight chunk of the other rank), with oracle pools filled by the oracle's own store and denoise
    passes: flow part of x0 within relative L2 1e-2 for every pass."""
    import exchange_model as em
    from waveforcing_amd.wavefront import WavefrontDenoiser

    dim, heads, ffn, layers, H, W = 256, 2, 512, 2, 16, 16
    hp, wp, npb, rf, window, n_chunks = H // 2, W // 2, 3, 2, 15, 4
    page = hp * wp
    T = npb * page
    bparams, dparams, _, ctx = _dit_case(dim, heads, ffn, layers, H, W, seed=61)
    blocks = [QuantizedWanBlock(p, heads, DEV) for p in bparams]
    dit = QuantizedWanDiT(dparams, QuantizedWanStack(blocks, PagedExchange(layers, heads, page, npb, window,
                                                                            rf_step=rf, device=DEV)))
    dit.set_text(ctx.to(DEV))
    record = []
    real_tick = dit.tick

    def spy(plan, inputs, concurrent=False):
        ins = {k: (lat.detach().cpu().clone(), float(t)) for k, (lat, t) in inputs.items()}
        out = real_tick(plan, inputs, concurrent=concurrent)
        record.append((plan, ins, {r: x0.detach().cpu().clone() for r, x0 in out.items()}))
        return out

    dit.tick = spy
    noise = torch.randn((1, 16, npb * n_chunks, H, W), generator=torch.Generator().manual_seed(62)).to(BF16)
    WavefrontDenoiser(dit, steps=(1000, 500)).generate(noise.to(DEV))
    torch.cuda.synchronize()
    assert len(record) == n_chunks + rf

    oemb = od.text_embed(dparams, ctx)
    otext = [ob.text_kv(p, oemb, heads) for p in bparams]
    sched = FlowMatchSchedule()
    pk = [okv.new_pool(npb * n_chunks, page, heads, 128) for _ in range(layers)]
    pv = [okv.new_pool(npb * n_chunks, page, heads, 128) for _ in range(layers)]

    def pages(c):
        return list(range(npb * c, npb * c + npb))

    clean, anchor_ku, checked, moved = [], [None] * layers, 0, False
    for plan, ins, outs in record:
        for r, c, csf, qf in em.passes(plan, rf, npb):
            lat, t = ins["store" if r == rf else r]
            anchor, start, ids = em.context(clean, plan, r, csf, qf, window, npb, rf)
            moved |= anchor is not None and start != anchor * npb

            def stack_fn(xs, e0):
                x = xs
                for L, p in enumerate(bparams):
                    if anchor is not None:
                        ang = ob.rope_angles(npb, hp, wp, start)
                        ak = ob.rope_apply_table(anchor_ku[L], torch.cos(ang).float(), torch.sin(ang).float())
                        okv.pack(ak, pages(anchor), page, *pk[L])
                    x, ku = ob.block_forward(p, x, e0, (npb, hp, wp), c * npb, pk[L], pv[L],
                                             [q for i in ids for q in pages(i)], pages(c), len(ids) * T, page,
                                             *otext[L], heads, return_unroped_k=True)
                    if r == rf and not clean:
                        anchor_ku[L] = ku
                return x

            want = od.dit_forward(dparams, stack_fn, lat[0], t, od.sigma_x0(sched.sigmas, sched.timesteps, t)).double()
            if r == rf:
                continue
            got = outs[r][0].double()
            xt = lat[0].permute(1, 0, 2, 3).double()
            rel = (((got - xt) - (want - xt)).norm() / (want - xt).norm()).item()
            print(f"tick {plan.tick} rank {r} chunk {c} t={t:.1f}: {len(ids)} context chunks, flow rel L2 {rel:.2e}")
            assert rel <= 1e-2
            checked += 1
        if plan.store_active:
            clean = em.keep_last(clean + [plan.tick - rf])
    assert checked == n_chunks * rf
    assert moved
