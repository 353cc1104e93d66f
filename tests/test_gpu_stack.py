"""GPU parity of the block stack driven through the paged exchange.

* Replay: a stack of 2 layers runs a denoise step and a store pass for each
  of chunks 0..9 (the clean list grows past the working set, then wraps at
  anchor + last 7, and slots are recycled).  A hand-written replay with the
  same blocks, a pool of its own (one fixed page range per chunk, no
  recycling) and a list model of the clean list (anchor re-RoPEd to
  ``csf - wflen - npb``, working set, chunk: common.py:70-114) must give the
  same hidden states, bit for bit, at every step.
* Oracle: stores of chunks 0..3 and a denoise step of chunk 4, which
  re-RoPEs the anchor to frame 3, against the CPU block oracle chained over
  the layers with its own pools and clean list.  Bar as for one block
  (relative L2 <= 1e-2, max |diff| <= 5e-2 * max |x|), since every input x
  is fresh and only the context carries differences between the two sides.
"""

import pytest
import torch

from oracle import block as ob
from oracle import kv as okv
from waveforcing_amd import exchange as ex
from waveforcing_amd import rope
from waveforcing_amd.block import QuantizedWanBlock, random_block_params
from waveforcing_amd.kv import Fp8PagePool
from waveforcing_amd.stack import QuantizedWanStack

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
DIM, HEADS, FFN = 256, 2, 512
NPB, HT, WD = 3, 8, 8              # 64-token pages: the attention kernel's key tile
PAGE = HT * WD
T = NPB * PAGE
WINDOW = 12        # (12 - 3 - 3) // 3 = 2 working chunks
LAYERS = 2


def _params():
    return [random_block_params(DIM, FFN, seed=70 + i) for i in range(LAYERS)]


def _inputs(c, store):
    g = torch.Generator().manual_seed(1000 + 2 * c + int(store))
    x = torch.randn((T, DIM), generator=g).to(torch.bfloat16)
    e = (torch.randn((NPB, 6, DIM), generator=g) * 0.1).to(torch.bfloat16)
    return x, e


def _text():
    return torch.randn((24, DIM), generator=torch.Generator().manual_seed(9)).to(torch.bfloat16)


def _stack(params):
    blocks = [QuantizedWanBlock(p, HEADS, DEV) for p in params]
    xch = ex.PagedExchange(LAYERS, HEADS, PAGE, NPB, WINDOW, device=DEV)
    st = QuantizedWanStack(blocks, xch)
    st.set_text(_text().to(DEV))
    return st


def _list_context(clean, csf, qf=NPB):
    """(anchor cid or None, anchor rope start, working cids) of the clean list model."""
    if not clean:
        return None, None, []
    _, n_w = ex.anchor_and_working(len(clean), ex.working_chunks(WINDOW, qf, NPB))
    working = clean[len(clean) - n_w:] if n_w else []
    return clean[0], ex.anchor_rope_start(csf, len(working), NPB), working


def _keep_last(clean):
    return clean[:1] + clean[-7:] if len(clean) > 8 else clean


def _pages(c):
    return list(range(NPB * c, NPB * c + NPB))


@pytest.mark.parametrize("qf", [NPB, 2 * NPB])   # one query chunk (2 working chunks) or two (1)
def test_stack_equals_manual_replay_over_ten_chunks(qf):
    params = _params()
    st = _stack(params)
    blocks = st.blocks
    n_chunks = 10
    own_pages = _pages(n_chunks)                      # the denoise step's own pages
    pools = [Fp8PagePool(NPB * (n_chunks + 1), HEADS, 128, PAGE, DEV) for _ in range(LAYERS)]
    text = [b.text_kv(_text().to(DEV)) for b in blocks]
    clean = [[] for _ in range(LAYERS)]
    anchor_ku = [None] * LAYERS
    for c in range(n_chunks):
        csf = c * NPB
        cos, sin = rope.cos_sin(NPB, HT, WD, csf, device=DEV)
        for store in (False, True):
            x, e = _inputs(c, store)
            q = NPB if store else qf     # store passes carry one chunk (paged.py:257-310)
            got = st.forward_chunk(x.to(DEV).clone(), e.to(DEV), c, HT, WD, store=store, query_frames=q)
            want = x.to(DEV).clone()
            for L, blk in enumerate(blocks):
                pool = pools[L]
                anchor, start, working = _list_context(clean[L], csf, q)
                ctx_pages = []
                if anchor is not None:
                    acos, asin = rope.cos_sin(NPB, HT, WD, start, device=DEV)
                    pool.pack(anchor_ku[L], None, pool.page_table(_pages(anchor)), rope=(acos, asin))
                    ctx_pages = _pages(anchor) + [p for w in working for p in _pages(w)]
                own = _pages(c) if store else own_pages
                ku = torch.empty_like(want) if store and not clean[L] else None
                blk.forward(want, e.to(DEV), cos, sin, pool, pool.page_table(ctx_pages + own), pool.page_table(own),
                            len(ctx_pages) * PAGE + T, text[L], unroped_k_out=ku)
                if store:
                    if ku is not None:
                        anchor_ku[L] = ku.view(T, HEADS, 128).clone()
                    clean[L] = _keep_last(clean[L] + [c])
            assert torch.equal(got, want), f"chunk {c} store={store}"
        assert [[p.cid for p in lst] for lst in st.exchange.clean] == clean
    # every slot is back on a free list or in a clean list
    for L in range(LAYERS):
        held = sorted(st.exchange._free[L] + [p.slot for p in st.exchange.clean[L]])
        assert held == list(range(st.exchange.n_slots))


def test_stack_matches_oracle_chain_with_anchor_rerope():
    params = _params()
    st = _stack(params)
    ctx_text = _text()
    otext = [ob.text_kv(p, ctx_text, HEADS) for p in params]
    P = NPB * 6
    own_pages = _pages(5)
    pk = [okv.new_pool(P, PAGE, HEADS, 128) for _ in range(LAYERS)]
    pv = [okv.new_pool(P, PAGE, HEADS, 128) for _ in range(LAYERS)]
    clean = [[] for _ in range(LAYERS)]
    anchor_ku = [None] * LAYERS
    steps = [(c, True) for c in range(4)] + [(4, False)]
    for c, store in steps:
        x, e = _inputs(c, store)
        got = st.forward_chunk(x.to(DEV).clone(), e.to(DEV), c, HT, WD, store=store).cpu().double()
        ref = x
        csf = c * NPB
        for L, p in enumerate(params):
            anchor, start, working = _list_context(clean[L], csf)
            ctx_pages = []
            if anchor is not None:
                ang = ob.rope_angles(NPB, HT, WD, start)
                ak = ob.rope_apply_table(anchor_ku[L], torch.cos(ang).float(), torch.sin(ang).float())
                okv.pack(ak, _pages(anchor), PAGE, *pk[L])
                ctx_pages = _pages(anchor) + [q for w in working for q in _pages(w)]
            own = _pages(c) if store else own_pages
            ref, ku = ob.block_forward(p, ref, e, (NPB, HT, WD), csf, pk[L], pv[L], ctx_pages + own, own,
                                       len(ctx_pages) * PAGE + T, PAGE, *otext[L], HEADS, return_unroped_k=True)
            if store:
                if not clean[L]:
                    anchor_ku[L] = ku
                clean[L] = _keep_last(clean[L] + [c])
        if c == 4:
            assert _list_context(clean[0], csf)[1] == 3   # the anchor really moved
        ref = ref.double()
        rel = ((got - ref).norm() / ref.norm()).item()
        mx = (got - ref).abs().max().item()
        print(f"chunk {c} store={store}: rel L2 {rel:.3e}, max abs {mx:.3e}, max|x| {ref.abs().max().item():.2f}")
        assert rel <= 1e-2
        assert mx <= 5e-2 * ref.abs().max().item()


def test_stack_releases_slots_when_a_layer_fails():
    st = _stack(_params())
    x, _ = _inputs(0, True)
    e5 = torch.zeros((5, 6, DIM), dtype=torch.bfloat16, device=DEV)   # 192 tokens do not split into 5 frames
    with pytest.raises(ValueError, match="5 frames"):
        st.forward_chunk(x.to(DEV), e5, 0, HT, WD, store=True)
    assert all(len(f) == st.exchange.n_slots for f in st.exchange._free) and not any(st.exchange.clean)
    with pytest.raises(ValueError, match="5 frames"):
        st.forward_chunk(x.to(DEV), e5, 0, HT, WD, store=False)
    assert all(len(f) == st.exchange.n_slots for f in st.exchange._free)
