"""Host logic of the single-GPU paged exchange (no GPU): the slot geometry of
wave_rt/denoiser/exchange/paged.py:161-190 and common.py:70-91, and the clean
list rule of common.py:110-114 (anchor + the last 7), checked against values
worked out by hand from those formulas."""

import pytest

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


def test_clean_list_keeps_anchor_and_last_seven_and_recycles_slots():
    x = ex.PagedExchange(n_layers=1, n_heads=1, tokens_per_frame=16, device="cpu")
    for cid in range(12):
        slot = x.reserve(0)
        x.append_clean(0, ex.CleanPage(cid=cid, slot=slot, ku=object() if cid == 0 else None))
    assert [p.cid for p in x.clean[0]] == [0, 5, 6, 7, 8, 9, 10, 11]
    used = {p.slot for p in x.clean[0]}
    assert len(used) == 8 and not (used & set(x._free[0]))
    assert len(x._free[0]) == x.n_slots - 8


def test_first_clean_chunk_must_carry_its_unrotated_key():
    x = ex.PagedExchange(n_layers=1, n_heads=1, tokens_per_frame=16, device="cpu")
    with pytest.raises(RuntimeError, match="anchor"):
        x.append_clean(0, ex.CleanPage(cid=0, slot=x.reserve(0)))


def test_slots_run_out_loudly():
    x = ex.PagedExchange(n_layers=1, n_heads=1, tokens_per_frame=16, n_inflight=0, device="cpu")
    for _ in range(x.n_slots):
        x.reserve(0)
    with pytest.raises(RuntimeError, match="no free slot"):
        x.reserve(0)


def test_denoise_step_must_release_its_slots_before_the_next():
    x = ex.PagedExchange(n_layers=1, n_heads=1, tokens_per_frame=16, device="cpu")
    x.make_denoise_exch(0)
    x._denoise_slots[0] = x.reserve(0)   # as the closure does on its first call
    with pytest.raises(RuntimeError, match="finish_denoise"):
        x.make_denoise_exch(3)
    x.finish_denoise()
    x.make_denoise_exch(3)


def test_anchor_promotion_needs_the_unrotated_key():
    x = ex.PagedExchange(n_layers=1, n_heads=1, tokens_per_frame=16, device="cpu")
    with pytest.raises(RuntimeError, match="unroped_key"):
        x.promote({0: (x.reserve(0), None)}, cid=0)


def test_layer_context_holds_one_slot_per_layer_and_pass():
    x = ex.PagedExchange(n_layers=2, n_heads=1, tokens_per_frame=16, device="cpu")
    # store pass of the first chunk: no clean chunks yet, the context is the chunk itself
    store_kv = {}
    pool, ctx, own, n_ctx = x.layer_context(0, 0, 3, 4, 4, store_kv)
    assert pool is x.pools[0] and n_ctx == x.T and len(own) == 3 and ctx.host == own.host
    slot = store_kv[0][0]
    assert own.host == x.slot_pages(slot)
    # a second call of the same layer in the same pass reuses the slot
    assert x.layer_context(0, 0, 3, 4, 4, store_kv)[2].host == own.host
    x.layer_context(1, 0, 3, 4, 4, store_kv)
    assert sorted(store_kv) == [0, 1] and len(x._free[0]) == x.n_slots - 1
    x.abort_store(store_kv)
    assert not store_kv and len(x._free[0]) == x.n_slots and len(x._free[1]) == x.n_slots
    # denoise pass: slots held until finish_denoise
    a = x.layer_context(0, 3, 3, 4, 4)[2].host
    assert x.layer_context(0, 3, 3, 4, 4)[2].host == a and len(x._free[0]) == x.n_slots - 1
    with pytest.raises(RuntimeError, match="finish_denoise"):
        x.make_denoise_exch(3)
    x.finish_denoise()
    assert len(x._free[0]) == x.n_slots
