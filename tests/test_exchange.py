"""Host logic of the single-GPU paged exchange (no GPU).

Checked against values worked out by hand from the reference's formulas and
against a list model written from them:

* the tick schedule of wave_rt/denoiser/engine.py:214-219,300-311 (active
  ranks, store activity, tick_csf, tick_qf);
* the denoise slot geometry of paged.py:161-190 (naw, live, in-flight order
  ``base_infl + #{n in act: m <= n < r}``, active_slots <= Wmax) and the
  store context of common.py:93-107;
* the clean list rule of common.py:110-114 (anchor + the last 7) and the
  clean length the reference expects at each tick, ``min(8, tick - store_rank)``;
* the 90 %-of-free-memory guard of paged.py:35-42.
"""

import pytest
import torch

from waveforcing_amd import exchange as ex


def test_working_chunks_examples():
    # 21-frame window, 3-frame chunks: one query chunk leaves (21 - 3 - 3) // 3 = 5 working chunks
    assert ex.working_chunks(21, 3, 3) == 5
    # four in-flight query chunks (rf_step 4): (21 - 12 - 3) // 3 = 2
    assert ex.working_chunks(21, 12, 3) == 2
    # window too small: clamps at zero
    assert ex.working_chunks(6, 6, 3) == 0
    assert ex.working_chunks(24, 3, 3) == 6


@pytest.mark.parametrize("clean_len,wmax,want", [
    (0, 5, (0, 0)), (1, 5, (1, 0)), (3, 5, (1, 2)), (8, 5, (1, 5)), (8, 0, (1, 0)), (2, 0, (1, 0)),
])
def test_anchor_and_working(clean_len, wmax, want):
    assert ex.anchor_and_working(clean_len, wmax) == want


def test_anchor_rope_start():
    # chunk 6 (frame 18) with 5 working chunks: the anchor sits at frames 0..2
    assert ex.anchor_rope_start(18, 5, 3) == 0
    # chunk 9 (frame 27): 27 - 15 - 3 = 9, just before the working set at frames 12..26
    assert ex.anchor_rope_start(27, 5, 3) == 9


@pytest.mark.parametrize("tick,act,store,csf,qf", [
    (0, [0], False, 0, 3),             # only rank 0 has a chunk
    (3, [0, 1, 2, 3], False, 0, 12),   # all four denoise ranks, store rank still idle (3 - 4 < 0)
    (4, [0, 1, 2, 3], True, 3, 12),    # steady state: oldest in-flight chunk is 4 - 3 = 1
    (10, [1, 2, 3], True, 21, 9),      # rank 0 ran out of chunks (10 >= 10); oldest is 10 - 3 = 7
    (13, [], True, 0, 0),              # only the store rank, storing chunk 9
])
def test_tick_plan_matches_engine_schedule(tick, act, store, csf, qf):
    p = ex.tick_plan(tick, rf_step=4, num_chunks=10, frames_per_chunk=3)
    assert (p.act_ranks, p.store_active, p.csf, p.qf) == (act, store, csf, qf)


def test_inflight_order_is_the_reference_slot_index():
    act = [0, 1, 2, 3]
    for m in act:
        order = ex.inflight_order(m, act)
        # producer r > m writes at base_infl + #{n in act: m <= n < r}; the consumer itself sits at base_infl
        for r in act:
            if r >= m:
                assert order.index(r) == sum(1 for n in act if m <= n < r)
    assert ex.inflight_order(1, [1, 2, 3]) == [1, 2, 3]
    assert ex.inflight_order(2, [0, 1, 2, 3]) == [2, 3]


def _list_context(clean, plan, rank, rf_step, window, npb):
    """Chunk ids of a context from the reference's formulas (paged.py:161-190, common.py:70-107)."""
    if rank is None:   # store pass of chunk plan.tick - rf_step
        wmax = ex.working_chunks(window, npb, npb)
    else:
        wmax = max(0, (window - len(plan.act_ranks) * npb - npb) // npb)
    ids = []
    if clean:
        naw = 1 + min(wmax, len(clean) - 1)
        ids = [clean[0]] + (clean[1:][-(naw - 1):] if naw > 1 else [])
    if rank is None:
        return ids + [plan.tick - rf_step]
    if plan.store_active:
        ids.append(plan.tick - rf_step)
    return ids + [plan.tick - n for n in ex.inflight_order(rank, plan.act_ranks)]


@pytest.mark.parametrize("rf_step,window,num_chunks", [(4, 21, 14), (3, 21, 12), (1, 12, 12), (2, 18, 9)])
def test_tick_contexts_follow_the_reference_geometry(rf_step, window, num_chunks):
    npb, L = 3, 2
    x = ex.PagedExchange(n_layers=L, n_heads=1, tokens_per_frame=16, frames_per_chunk=npb, max_attn_frames=window,
                         rf_step=rf_step, device="cpu")
    clean_model = []
    longest = 0
    for t in range(num_chunks + rf_step):
        plan = x.begin_tick_at(t, num_chunks)
        # the reference's expected clean length at this tick (paged.py:164, store_rank = rf_step)
        assert len(x.clean[0]) == min(8, max(0, t - rf_step)) == len(clean_model)
        slot_chunk = {L_: {c.slot: c.cid for c in x.clean[L_]} for L_ in range(L)}
        passes = ([(None, x.store_pass())] if plan.store_active else []) + \
                 [(r, x.denoise_pass(r)) for r in sorted(plan.act_ranks, reverse=True)]
        for rank, p in passes:
            assert p.chunk == t - (rf_step if rank is None else rank)
            for layer in range(L):
                slots, own = x.context_slots(layer, p)
                slot_chunk[layer][own] = p.chunk
                got = [slot_chunk[layer][s] for s in slots]
                assert got == _list_context(clean_model, plan, rank, rf_step=rf_step, window=window, npb=npb)
                assert len(slots) <= x.n_slots
                longest = max(longest, len(slots))
        x.end_tick()
        if plan.store_active:
            clean_model.append(t - rf_step)
            if len(clean_model) > 8:
                clean_model = clean_model[:1] + clean_model[-7:]
        for layer in range(L):
            assert [c.cid for c in x.clean[layer]] == clean_model
            assert len(x._free[layer]) == x.n_slots - len(clean_model)
    if (rf_step, window) == (4, 21):
        # steady state: anchor + 2 working + live + self + 3 in-flight = 8 chunks (37440 keys at 4680 tokens)
        assert longest == 8


def test_denoise_ranks_must_run_after_the_store_pass_and_from_the_highest_down():
    x = ex.PagedExchange(n_layers=1, n_heads=1, tokens_per_frame=16, rf_step=2, device="cpu")
    x.begin_tick_at(2, num_chunks=5)                  # ranks 0 and 1 active, store stores chunk 0
    with pytest.raises(RuntimeError, match="store pass"):
        x.context_slots(0, x.denoise_pass(1))
    x.context_slots(0, x.store_pass())
    with pytest.raises(RuntimeError, match="rank 1 has not published"):
        x.context_slots(0, x.denoise_pass(0))
    x.abort_tick()
    assert len(x._free[0]) == x.n_slots and not x.clean[0]


def test_idle_passes_and_unfinished_ticks_are_refused():
    x = ex.PagedExchange(n_layers=1, n_heads=1, tokens_per_frame=16, rf_step=4, device="cpu")
    with pytest.raises(RuntimeError, match="no tick"):
        x.store_pass()
    x.begin_tick_at(0, num_chunks=3)
    with pytest.raises(RuntimeError, match="idle"):
        x.store_pass()
    with pytest.raises(RuntimeError, match="idle"):
        x.denoise_pass(1)
    with pytest.raises(RuntimeError, match="has not ended"):
        x.begin_tick_at(1, num_chunks=3)
    x.end_tick()
    x.begin_tick_at(1, num_chunks=3)


def test_store_pass_must_publish_every_layer_before_promotion():
    x = ex.PagedExchange(n_layers=2, n_heads=1, tokens_per_frame=16, rf_step=1, device="cpu")
    x.begin_tick_at(1, num_chunks=3)
    x.context_slots(0, x.store_pass())
    with pytest.raises(RuntimeError, match="every layer"):
        x.end_tick()
    x.abort_tick()
    assert all(len(f) == x.n_slots for f in x._free)


def test_clean_list_keeps_anchor_and_last_seven_and_recycles_slots():
    x = ex.PagedExchange(n_layers=1, n_heads=1, tokens_per_frame=16, device="cpu")
    for cid in range(12):
        x.append_clean(0, ex.CleanPage(cid=cid, slot=x.reserve(0)))
    assert [p.cid for p in x.clean[0]] == [0, 5, 6, 7, 8, 9, 10, 11]
    used = {p.slot for p in x.clean[0]}
    assert len(used) == 8 and not (used & set(x._free[0]))
    assert len(x._free[0]) == x.n_slots - 8


def test_slots_run_out_loudly():
    x = ex.PagedExchange(n_layers=1, n_heads=1, tokens_per_frame=16, rf_step=1, device="cpu")
    for _ in range(x.n_slots):
        x.reserve(0)
    with pytest.raises(RuntimeError, match="no free slot"):
        x.reserve(0)


def test_capacity_guard_refuses_pools_above_ninety_percent_of_free(monkeypatch):
    monkeypatch.setattr(torch.cuda, "mem_get_info", lambda device=None: (1000, 4000))
    ex.check_capacity(900, "cuda:0")
    with pytest.raises(RuntimeError, match="90% of free"):
        ex.check_capacity(901, "cuda:0")
    with pytest.raises(RuntimeError, match="90% of free"):
        ex.PagedExchange(n_layers=30, n_heads=12, tokens_per_frame=1560, device="cuda:0")


def test_reset_starts_a_new_stream_with_the_same_contexts():
    """After reset (the fresh clean lists of each run of the tick loop, engine.py:294) a second stream sees
    the same slot contexts as the first; a reset inside a tick is refused."""
    npb, L, rf_step, num_chunks = 3, 2, 4, 10
    x = ex.PagedExchange(n_layers=L, n_heads=1, tokens_per_frame=16, frames_per_chunk=npb, max_attn_frames=21,
                         rf_step=rf_step, device="cpu")

    def stream():
        seen = []
        for t in range(num_chunks + rf_step):
            plan = x.begin_tick_at(t, num_chunks)
            passes = ([x.store_pass()] if plan.store_active else []) + \
                     [x.denoise_pass(r) for r in sorted(plan.act_ranks, reverse=True)]
            for p in passes:
                for layer in range(L):
                    slots, own = x.context_slots(layer, p)
                    seen.append((t, p.kind, p.chunk, layer, tuple(slots), own))
            x.end_tick()
        return seen

    first = stream()
    assert len(x.clean[0]) == 8
    x.begin_tick_at(0, num_chunks)
    with pytest.raises(RuntimeError, match="tick is in progress"):
        x.reset()
    x.abort_tick()
    x.reset()
    assert all(not c for c in x.clean) and all(len(f) == x.n_slots for f in x._free)
    assert stream() == first


def test_anchor_rotation_follows_the_pass_grid(monkeypatch):
    """The anchor pages are re-rotated when a pass has another (height, width) of the same token count and
    the same rope start: the rotation in place is keyed by (start, height, width), not by the start alone."""
    x = ex.PagedExchange(n_layers=1, n_heads=1, tokens_per_frame=16, frames_per_chunk=3, max_attn_frames=21,
                         rf_step=1, device="cpu")
    calls = []
    monkeypatch.setattr(x.pool, "pack", lambda *a, **k: calls.append(k["rope"][0].clone()))
    x.begin_tick_at(1, num_chunks=4)                       # the store pass of chunk 0: it becomes the anchor
    x.context_slots(0, x.store_pass())
    assert x.anchor_ku_out(0) is not None
    x.end_tick()
    x.begin_tick_at(2, num_chunks=4)
    p = x.denoise_pass(0)
    x.prepare_pass(p, 4, 4)
    x.prepare_pass(p, 4, 4)                                 # memo: no second rotation
    x.prepare_pass(p, 2, 8)                                 # another grid, same start and token count
    x.prepare_pass(p, 4, 4)
    x.abort_tick()
    assert len(calls) == 3
    assert not torch.equal(calls[0], calls[1]) and torch.equal(calls[0], calls[2])


def test_table_cache_is_only_cleared_between_ticks(monkeypatch):
    monkeypatch.setattr(ex, "TABLE_CACHE_MAX", 4)
    x = ex.PagedExchange(n_layers=1, n_heads=1, tokens_per_frame=16, rf_step=1, device="cpu")
    x.begin_tick_at(1, num_chunks=3)
    tabs = [x.table(0, [s]) for s in range(x.n_slots)]
    assert len(x._tables) == x.n_slots > 4              # inside a tick nothing is dropped
    assert all(x.table(0, [s]) is t for s, t in enumerate(tabs))
    x.abort_tick()
    x.begin_tick_at(1, num_chunks=3)
    assert not x._tables
    x.abort_tick()
