"""A list model of the reference's per-pass contexts (test helper, no GPU).

For a tick's pass it gives the chunk ids in the reference's order and the anchor's re-RoPE start
(paged.py:161-190,236-247; common.py:70-91): a store pass sees anchor + working + itself, a denoise
pass of rank r anchor + working + the live stored chunk + itself + the in-flight chunks of the other
ranks (inflight_order).  The clean list keeps the anchor and the last 7 chunks (common.py:110-114).
"""

from waveforcing_amd import exchange as ex


def passes(plan, rf: int, npb: int):
    """(rank, chunk, csf, qf) of a tick's passes in execution order; rank ``rf`` is the store rank."""
    out = [(rf, plan.tick - rf, (plan.tick - rf) * npb, npb)] if plan.store_active else []
    return out + [(r, plan.tick - r, plan.csf, plan.qf) for r in sorted(plan.act_ranks, reverse=True)]


def context(clean, plan, rank, csf, qf, window: int, npb: int, rf: int):
    """(anchor chunk or None, its rope start, context chunk ids in the reference's order)."""
    anchor, start, ids = None, None, []
    if clean:
        _, n_w = ex.anchor_and_working(len(clean), ex.working_chunks(window, qf, npb))
        working = clean[len(clean) - n_w:] if n_w else []
        anchor, start = clean[0], ex.anchor_rope_start(csf, len(working), npb)
        ids = [anchor] + working
    if rank == rf:
        return anchor, start, ids + [plan.tick - rf]
    if plan.store_active:
        ids.append(plan.tick - rf)
    return anchor, start, ids + [plan.tick - n for n in ex.inflight_order(rank, plan.act_ranks)]


def keep_last(clean):
    return clean[:1] + clean[-7:] if len(clean) > 8 else clean
