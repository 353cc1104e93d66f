"""GPU parity of the block stack driven tick by tick through the paged exchange.

The wavefront's schedule (wave_rt/denoiser/engine.py:300-420) at rf_step 2:
each tick runs the store rank's pass and the active denoise ranks' passes.

* Replay: ticks 0..10 of a 9-chunk stream through a 2-layer stack (the clean
  list grows past the working set and wraps at anchor + last 7, slots are
  recycled).  A hand-written replay with the same blocks, a pool of its own
  (one fixed page range per chunk, no recycling) and a list model of the
  reference's contexts (store: anchor + working + self; denoise: anchor +
  working + live + self + in-flight n > r, paged.py:161-190, with the anchor
  re-RoPEd to ``csf - wflen - npb``, common.py:70-91) must give the same
  hidden states, bit for bit, for every pass.
* Oracle: ticks 0..5 of a 4-chunk stream against the CPU block oracle
  chained over the layers with its own pools and the same list model
  (anchor re-RoPE included).  Bar as for one block (relative L2 <= 1e-2,
  max |diff| <= 5e-2 * max |x|), since every input x is fresh and only the
  context carries differences between the two sides.
* A failing layer returns every slot of the tick and promotes nothing.
* 14B composition: a 40-layer 14B stack's pass (each block's last gated
  residual fused into the next block's first LayerNorm) equals 40 plain
  single-block forward calls over the same contexts bit for bit, on a
  denoise pass over two stored chunks; and a 3-layer 14B-width stack equals
  the CPU oracle chained over its layers within the block bar.
"""

import pytest
import torch

import exchange_model as em
from oracle import block as ob
from oracle import kv as okv
from waveforcing_amd import exchange as ex
from waveforcing_amd import rope
from waveforcing_amd.block import QuantizedWanBlock, random_block_params
from waveforcing_amd.kv import Fp8PagePool
from waveforcing_amd.stack import QuantizedWanStack

H14, W14 = 30, 52        # a 4680-token chunk of 1560-token frames

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
DIM, HEADS, FFN = 256, 2, 512
NPB, HT, WD = 3, 8, 8              # 64-token pages: the attention kernel's key tile
PAGE = HT * WD
T = NPB * PAGE
WINDOW = 15        # one query chunk: (15 - 3 - 3) // 3 = 3 working chunks; two (rf_step 2): 2
RF = 2
LAYERS = 2


def _params():
    return [random_block_params(DIM, FFN, seed=70 + i) for i in range(LAYERS)]


def _inputs(t, rank):
    """Seeded hidden states and modulation of a pass (rank RF = the store rank)."""
    g = torch.Generator().manual_seed(1000 + 10 * t + rank)
    x = torch.randn((T, DIM), generator=g).to(torch.bfloat16)
    e = (torch.randn((NPB, 6, DIM), generator=g) * 0.1).to(torch.bfloat16)
    return x, e


def _text():
    return torch.randn((24, DIM), generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)


def _stack(params):
    blocks = [QuantizedWanBlock(p, HEADS, DEV) for p in params]
    xch = ex.PagedExchange(LAYERS, HEADS, PAGE, NPB, WINDOW, rf_step=RF, device=DEV)
    st = QuantizedWanStack(blocks, xch)
    st.set_text(_text().to(DEV))
    return st


def _pages(c):
    return list(range(NPB * c, NPB * c + NPB))


def _passes(plan):
    return em.passes(plan, RF, NPB)


def _context(clean, plan, rank, csf, qf):
    return em.context(clean, plan, rank, csf, qf, WINDOW, NPB, RF)


_keep_last = em.keep_last


def test_stack_ticks_equal_manual_replay():
    params = _params()
    st = _stack(params)
    blocks = st.blocks
    n_chunks = 9
    pools = [Fp8PagePool(NPB * n_chunks, HEADS, 128, PAGE, DEV) for _ in range(LAYERS)]
    text = [b.text_kv(_text().to(DEV)) for b in blocks]
    clean, anchor_ku = [], [None] * LAYERS
    for t in range(n_chunks + RF):
        plan = ex.tick_plan(t, RF, n_chunks, NPB)
        ins = {(r if r != RF else "store"): _inputs(t, r) for r, *_ in _passes(plan)}
        got = {k: (x.to(DEV).clone(), e.to(DEV)) for k, (x, e) in ins.items()}
        st.tick(plan, got, HT, WD)
        for r, c, csf, qf in _passes(plan):
            x, e = ins["store" if r == RF else r]
            want = x.to(DEV).clone()
            cos, sin = rope.cos_sin(NPB, HT, WD, c * NPB, device=DEV)
            anchor, start, ids = _context(clean, plan, r, csf, qf)
            for L, blk in enumerate(blocks):
                pool = pools[L]
                if anchor is not None:
                    acos, asin = rope.cos_sin(NPB, HT, WD, start, device=DEV)
                    pool.pack(anchor_ku[L], None, pool.page_table(_pages(anchor)), rope=(acos, asin))
                ku = torch.empty_like(want) if r == RF and not clean else None
                blk.forward(want, e.to(DEV), cos, sin, pool, pool.page_table([p for i in ids for p in _pages(i)]),
                            pool.page_table(_pages(c)), len(ids) * T, text[L], unroped_k_out=ku)
                if ku is not None:
                    anchor_ku[L] = ku.view(T, HEADS, 128).clone()
            assert torch.equal(got["store" if r == RF else r][0], want), f"tick {t} rank {r}"
        if plan.store_active:
            clean = _keep_last(clean + [t - RF])
        assert [[p.cid for p in lst] for lst in st.exchange.clean] == [clean] * LAYERS
    # every slot is back on a free list or in a clean list
    for L in range(LAYERS):
        held = sorted(st.exchange._free[L] + [p.slot for p in st.exchange.clean[L]])
        assert held == list(range(st.exchange.n_slots))


def test_stack_ticks_match_oracle_chain_with_anchor_rerope():
    params = _params()
    st = _stack(params)
    ctx_text = _text()
    otext = [ob.text_kv(p, ctx_text, HEADS) for p in params]
    n_chunks = 4
    pk = [okv.new_pool(NPB * n_chunks, PAGE, HEADS, 128) for _ in range(LAYERS)]
    pv = [okv.new_pool(NPB * n_chunks, PAGE, HEADS, 128) for _ in range(LAYERS)]
    clean, anchor_ku = [], [None] * LAYERS
    moved = False
    for t in range(n_chunks + RF):
        plan = ex.tick_plan(t, RF, n_chunks, NPB)
        ins = {(r if r != RF else "store"): _inputs(t, r) for r, *_ in _passes(plan)}
        got = {k: (x.to(DEV).clone(), e.to(DEV)) for k, (x, e) in ins.items()}
        st.tick(plan, got, HT, WD)
        for r, c, csf, qf in _passes(plan):
            x, e = ins["store" if r == RF else r]
            ref = x
            anchor, start, ids = _context(clean, plan, r, csf, qf)
            moved |= anchor is not None and start != anchor * NPB
            for L, p in enumerate(params):
                if anchor is not None:
                    ang = ob.rope_angles(NPB, HT, WD, start)
                    ak = ob.rope_apply_table(anchor_ku[L], torch.cos(ang).float(), torch.sin(ang).float())
                    okv.pack(ak, _pages(anchor), PAGE, *pk[L])
                ref, ku = ob.block_forward(p, ref, e, (NPB, HT, WD), c * NPB, pk[L], pv[L],
                                           [q for i in ids for q in _pages(i)], _pages(c), len(ids) * T, PAGE,
                                           *otext[L], HEADS, return_unroped_k=True)
                if r == RF and not clean:
                    anchor_ku[L] = ku
            out = got["store" if r == RF else r][0].cpu().double()
            ref = ref.double()
            rel = ((out - ref).norm() / ref.norm()).item()
            mx = (out - ref).abs().max().item()
            print(f"tick {t} rank {r} chunk {c}: {len(ids)} context chunks, rel L2 {rel:.3e}, max abs {mx:.3e}")
            assert rel <= 1e-2
            assert mx <= 5e-2 * ref.abs().max().item()
        if plan.store_active:
            clean = _keep_last(clean + [t - RF])
    assert moved   # some pass rotated the anchor away from its own position


def test_stack_tick_releases_slots_when_a_layer_fails():
    st = _stack(_params())
    x, _ = _inputs(0, 0)
    e5 = torch.zeros((5, 6, DIM), dtype=torch.bfloat16, device=DEV)   # 192 tokens do not split into 5 frames
    plan = ex.tick_plan(RF, RF, 4, NPB)                                 # store pass + ranks 0 and 1
    ins = {k: (x.to(DEV).clone(), e5) for k in ("store", 0, 1)}
    with pytest.raises(ValueError, match="5 frames"):
        st.tick(plan, ins, HT, WD)
    assert all(len(f) == st.exchange.n_slots for f in st.exchange._free) and not any(st.exchange.clean)
    with pytest.raises(ValueError, match="5 frames"):
        st.forward_chunk(x.to(DEV), e5, 0, HT, WD, store=False)
    assert all(len(f) == st.exchange.n_slots for f in st.exchange._free)


@pytest.mark.parametrize("rf_step,layers", [(2, 2), (4, 3)])
def test_concurrent_tick_wavefront_is_bit_identical(rf_step, layers):
    """The denoise ranks of each tick as a layer wavefront on one stream per rank (tick(concurrent=True))
    give the same hidden states, bit for bit, as the ranks one after another, over a whole stream of ticks
    (clean list filling, wrapping and slot recycling included), and leave the same clean lists."""
    params = [random_block_params(DIM, FFN, seed=170 + i) for i in range(layers)]
    window = 21 if rf_step == 4 else WINDOW

    def make():
        blocks = [QuantizedWanBlock(p, HEADS, DEV) for p in params]
        st = QuantizedWanStack(blocks, ex.PagedExchange(layers, HEADS, PAGE, NPB, window, rf_step=rf_step,
                                                        device=DEV))
        st.set_text(_text().to(DEV))
        return st

    seq, con = make(), make()
    n_chunks = 10
    for t in range(n_chunks + rf_step):
        plan = ex.tick_plan(t, rf_step, n_chunks, NPB)
        keys = (["store"] if plan.store_active else []) + list(plan.act_ranks)
        ins = {k: _inputs(t, rf_step if k == "store" else k) for k in keys}
        a = {k: (x.to(DEV), e.to(DEV)) for k, (x, e) in ins.items()}
        b = {k: (x.to(DEV), e.to(DEV)) for k, (x, e) in ins.items()}
        seq.tick(plan, a, HT, WD)
        con.tick(ex.tick_plan(t, rf_step, n_chunks, NPB), b, HT, WD, concurrent=True)
        torch.cuda.synchronize()
        for k in keys:
            assert torch.equal(a[k][0], b[k][0]), f"tick {t} pass {k}"
        assert [[p.cid for p in c] for c in seq.exchange.clean] == [[p.cid for p in c] for c in con.exchange.clean]
    for L in range(layers):
        assert sorted(con.exchange._free[L] + [p.slot for p in con.exchange.clean[L]]) == list(
            range(con.exchange.n_slots))


def test_wavefront_refuses_mixed_or_misordered_passes():
    st = _stack(_params())
    plan = ex.tick_plan(RF + 1, RF, 6, NPB)      # store pass + ranks 0 and 1
    st.exchange.begin_tick(plan)
    x, e = _inputs(0, 0)
    x, e = x.to(DEV), e.to(DEV)
    p1, p0 = st.exchange.denoise_pass(1), st.exchange.denoise_pass(0)
    with pytest.raises(ValueError, match="highest rank down"):
        st.run_wavefront([(x, e, p0), (x.clone(), e, p1)], HT, WD)
    with pytest.raises(ValueError, match="denoise passes"):
        st.run_wavefront([(x, e, st.exchange.store_pass())], HT, WD)
    st.exchange.abort_tick()


def _x14(seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((3 * H14 * W14, 5120), generator=g).to(torch.bfloat16)
    e = (torch.randn((3, 6, 5120), generator=g) * 0.1).to(torch.bfloat16)
    return x, e


def test_14b_forty_layer_pass_equals_single_block_calls():
    st = QuantizedWanStack.random("14b", seed=500, device=DEV, rf_step=4)
    assert len(st.blocks) == 40
    st.set_text(torch.randn((512, 5120), generator=torch.Generator().manual_seed(8)).to(torch.bfloat16).to(DEV))
    xch = st.exchange
    for c in range(2):
        x, e = _x14(600 + c)
        st.forward_chunk(x.to(DEV), e.to(DEV), c, H14, W14, store=True)
    x, e = _x14(610)
    x, e = x.to(DEV), e.to(DEV)
    plan = ex.TickPlan(2, [0], False, 2 * NPB, NPB)
    xch.begin_tick(plan)
    try:
        p = xch.denoise_pass(0)
        fused = x.clone()
        st.run_pass(fused, e, p, H14, W14)
        single = x.clone()
        cos, sin = rope.cos_sin(NPB, H14, W14, p.chunk * NPB, 128, device=DEV)
        n_ctx = set()
        for L, blk in enumerate(st.blocks):
            pool, ctx, own, n = xch.layer_context(L, p, H14, W14)
            n_ctx.add(n)
            blk.forward(single, e, cos, sin, pool, ctx, own, n, st.text_kv[L])
        torch.cuda.synchronize()
    finally:
        xch.abort_tick()
    print(f"context {sorted(n_ctx)} keys per layer; equal {(fused == single).double().mean().item():.6f}")
    assert n_ctx == {3 * 4680}     # anchor + working chunk + self
    assert torch.equal(fused, single)


def test_14b_three_layer_stack_matches_oracle_chain():
    dim, heads, ffn, layers = 5120, 40, 13824, 3
    params = [random_block_params(dim, ffn, seed=520 + i) for i in range(layers)]
    text = (torch.randn((512, dim), generator=torch.Generator().manual_seed(9))).to(torch.bfloat16)
    blocks = [QuantizedWanBlock(q, heads, DEV) for q in params]
    st = QuantizedWanStack(blocks, ex.PagedExchange(layers, heads, H14 * W14, NPB, 21, rf_step=4, device=DEV))
    st.set_text(text.to(DEV))
    x, e = _x14(620)
    out = st.forward_chunk(x.to(DEV).clone(), e.to(DEV), 0, H14, W14).cpu().double()
    del st, blocks
    torch.cuda.empty_cache()
    page = H14 * W14
    ref = x
    for L, q in enumerate(params):
        pk, pv = okv.new_pool(NPB, page, heads, 128), okv.new_pool(NPB, page, heads, 128)
        tk, tv = ob.text_kv(q, text, heads)
        ref = ob.block_forward(q, ref, e, (NPB, H14, W14), 0, pk, pv, [0, 1, 2], [0, 1, 2], NPB * page, page,
                               tk, tv, heads)
        print(f"oracle layer {L} done", flush=True)
    ref = ref.double()
    rel = ((out - ref).norm() / ref.norm()).item()
    mx = (out - ref).abs().max().item()
    print(f"3-layer 14B stack vs oracle chain: rel L2 {rel:.3e}, max abs {mx:.3e}, max|x| {ref.abs().max().item():.2f}")
    assert rel <= 1e-2
    assert mx <= 5e-2 * ref.abs().max().item()
