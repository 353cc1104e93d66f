"""Paged FP8 KV exchange of a whole wavefront on one GPU.

Restates the fixed-slot paged exchange of WaveRT
(wave_rt/denoiser/exchange/paged.py:13-310), its context assembly
(common.py:45-114) and the tick schedule that drives it
(wave_rt/denoiser/engine.py:214-219,300-311) over FP8 page pools, for a
wavefront whose ranks all run on this GPU:

* at tick t, denoise rank r (DMD step r, 0 <= r < rf_step) holds chunk t - r
  and the store rank (rf_step) re-runs chunk t - rf_step with clean context
  noise; ``act_ranks`` are the ranks with a chunk, ``tick_csf`` is the first
  latent frame of the oldest in-flight chunk and ``tick_qf`` the frames of all
  in-flight chunks (engine.py:300-311);
* the clean list per layer is the anchor (the first clean chunk) plus the
  last 7 clean chunks (``_append_clean_page``, common.py:110-114); the stored
  chunk joins it when the tick ends (engine.py:433-503);
* a denoise context is [anchor, working..., live, self, in-flight n > r ...]
  (``_make_denoise_exch_paged``, paged.py:161-190): the anchor re-RoPEd to
  ``tick_csf - wflen - npb``, the last ``wmax_chunks`` clean chunks with
  ``wmax_chunks = (max_attn_frames - len(act_ranks) * npb - npb) // npb``, the
  store rank's chunk of this tick when it is active, the rank's own chunk,
  then the chunks of the active ranks above it in ascending order (a producer
  r writes into consumer m's slot ``base_infl + #{n in act: m <= n < r}``);
* a store context is [anchor, working..., self] with the one-chunk geometry
  (``_assemble_store_context``, common.py:93-107);
* the closures keep the reference's keyword signature (paged.py:191-205).

One GPU runs the passes of a tick one after another: the store pass first (it
reads no in-flight chunk), then the denoise ranks from the highest down, so
every in-flight chunk a rank reads (n > r) is already in its slot -- the order
the reference's flag waits enforce across GPUs (paged.py:147-154,236-237).

The reference copies anchor, working set and self into fixed bf16 slab slots
every layer of every step (paged.py:215-237).  Here each chunk is quantized
into its pages once, when it is produced, and a context is a page table over
those pages.  Only the anchor's K is rewritten, once per pass geometry for
every layer in one launch (``wf_fp8_kv_pack_rope_tiled``), because its
rotation depends on the geometry; its V is packed once.

Pages: one pool holds every layer.  Layer L owns pages
[L * pages_per_layer, (L + 1) * pages_per_layer): ``n_slots`` chunk slots of
``frames_per_chunk`` pages (one latent frame per page) = 8 clean chunks + the
live chunk + rf_step in-flight chunks, the slab geometry
``Wmax = naw + 1 + rf_step`` of paged.py:26-29 with the clean list's 8 chunks
in place of ``naw``.  Attention reads a per-layer view of the pool, so each
view stays below the attention kernel's 2 GiB code-pool limit.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import rope
from .kv import Fp8PagePool, PagedKV, PageTable

MAX_CLEAN = 8  # anchor + the last 7 clean chunks (common.py:110-114)
TABLE_CACHE_MAX = 4096  # cached page tables, cleared between ticks once reached


def working_chunks(max_attn_frames: int, query_frames: int, frames_per_chunk: int) -> int:
    """Working-set size in chunks: ``wmax_chunks`` of common.py:75-76 and paged.py:166."""
    return max(0, (max_attn_frames - query_frames - frames_per_chunk) // frames_per_chunk)


def anchor_and_working(clean_len: int, wmax_chunks: int) -> tuple[int, int]:
    """(anchor count, working count) of a clean list of ``clean_len`` chunks (common.py:73-80)."""
    if clean_len == 0:
        return 0, 0
    return 1, min(wmax_chunks, clean_len - 1) if wmax_chunks > 0 else 0


def anchor_rope_start(chunk_start_frame: int, n_working: int, frames_per_chunk: int) -> int:
    """Latent frame the anchor is rotated to: ``csf - wflen - npb`` (common.py:81)."""
    return chunk_start_frame - n_working * frames_per_chunk - frames_per_chunk


def inflight_order(rank: int, act_ranks: list[int]) -> list[int]:
    """Ranks whose chunks follow the live chunk in rank ``rank``'s context: itself, then the active ranks
    above it in ascending order (the slot index base_infl + #{n in act: m <= n < r}, paged.py:181-190)."""
    return [rank] + sorted(n for n in act_ranks if n > rank)


def check_capacity(need_bytes: int, device) -> None:
    """Refuse pools above 90 % of the device's free memory, as ``_init_paged`` does (paged.py:35-42)."""
    device = torch.device(device)
    if device.type != "cuda":
        return
    free_b, _total = torch.cuda.mem_get_info(device)
    if need_bytes > free_b * 0.9:
        raise RuntimeError(f"[paged] FP8 KV pages {need_bytes / 2**30:.1f} GiB exceed 90% of free "
                           f"{free_b / 2**30:.1f} GiB")


@dataclass
class TickPlan:
    """Which passes run at one tick and the shared geometry of the denoise contexts (engine.py:300-311)."""

    tick: int
    act_ranks: list[int]   # denoise ranks with a chunk at this tick, ascending
    store_active: bool     # the store rank stores chunk tick - rf_step
    csf: int               # tick_csf: first latent frame of the oldest in-flight chunk
    qf: int                # tick_qf: latent frames of all in-flight chunks


def tick_plan(tick: int, rf_step: int, num_chunks: int, frames_per_chunk: int) -> TickPlan:
    """The reference's schedule at ``tick`` (``_act_denoise`` / ``_act_store``, engine.py:214-219,
    and the tick geometry, engine.py:307-311)."""
    act = [n for n in range(rf_step) if 0 <= tick - n < num_chunks]
    oldest = (tick - max(act)) if act else 0
    return TickPlan(tick, act, 0 <= tick - rf_step < num_chunks, oldest * frames_per_chunk,
                    len(act) * frames_per_chunk)


@dataclass
class Pass:
    """One chunk's forward through the layers within a tick."""

    kind: str      # "store" or "denoise"
    chunk: int     # chunk index (latent frames chunk * npb ...)
    rank: int      # the denoise rank, or rf_step for the store rank
    csf: int       # start frame of the pass's anchor/working geometry
    qf: int        # query frames of that geometry (sizes the working set)


@dataclass
class CleanPage:
    """One chunk of a layer's clean list and the slot holding its pages."""

    cid: int
    slot: int


class PagedExchange:
    """FP8 page slots of every layer, the clean lists, the tick's passes and the exchange closures."""

    def __init__(self, n_layers: int, n_heads: int, tokens_per_frame: int, frames_per_chunk: int = 3,
                 max_attn_frames: int = 21, head_dim: int = 128, rf_step: int = 4, device="cuda") -> None:
        if rf_step < 1:
            raise ValueError("rf_step must be >= 1")
        self.n_layers = n_layers
        self.n_heads = n_heads
        self.head_dim = head_dim
        self.npb = frames_per_chunk
        self.page_tokens = tokens_per_frame
        self.T = tokens_per_frame * frames_per_chunk
        self.max_attn_frames = max_attn_frames
        self.rf_step = rf_step
        self.device = torch.device(device)
        self.n_slots = MAX_CLEAN + 1 + rf_step
        self.pages_per_layer = self.n_slots * frames_per_chunk
        pages = n_layers * self.pages_per_layer
        check_capacity(Fp8PagePool.bytes_for(pages, n_heads, head_dim, tokens_per_frame)
                       + n_layers * self.T * n_heads * head_dim * 2, self.device)
        self.pool = Fp8PagePool(pages, n_heads, head_dim, tokens_per_frame, self.device)
        self.pools = [Fp8PagePool.view_of(self.pool, L * self.pages_per_layer, self.pages_per_layer)
                      for L in range(n_layers)]
        self.clean: list[list[CleanPage]] = [[] for _ in range(n_layers)]
        self._free: list[list[int]] = [list(range(self.n_slots)) for _ in range(n_layers)]
        self._tables: dict = {}
        # the anchor chunk's normalized, un-rotated K of every layer [Ln, T, H, D] (allocated with the first
        # store pass), and the anchor re-RoPE start its pages currently hold
        self.anchor_ku: torch.Tensor | None = None
        self._anchor_rot: tuple | None = None    # (rope_start, height, width) of the anchor pages' rotation
        self._plan: TickPlan | None = None
        self._store: Pass | None = None
        self._live: dict[int, int] = {}                                   # layer -> slot of the stored chunk
        self._inflight: list[dict[int, int]] = [{} for _ in range(n_layers)]  # layer -> {rank: slot}
        # per-pass memo of the host work every layer of a pass repeats: the pass whose anchor rotation is in
        # place, and the pass's clean-list positions of [anchor, working...] (equal on every layer)
        self._clean_version = 0
        self._prepared: tuple | None = None
        self._geometry: tuple | None = None

    # ---------------------------------------------------------------- slots
    def slot_pages(self, slot: int) -> list[int]:
        return [slot * self.npb + f for f in range(self.npb)]

    def table(self, layer: int, slots: list[int]) -> PageTable:
        """Page table (layer-local page ids) over ``slots`` of ``layer``, cached."""
        key = (layer, tuple(slots))
        t = self._tables.get(key)
        if t is None:
            t = self.pools[layer].page_table([p for s in slots for p in self.slot_pages(s)])
            self._tables[key] = t
        return t

    def reserve(self, layer: int) -> int:
        """Take a free slot of ``layer``."""
        if not self._free[layer]:
            raise RuntimeError(f"[paged] layer {layer}: no free slot ({self.n_slots} slots, "
                               f"{len(self.clean[layer])} clean)")
        return self._free[layer].pop(0)

    def release(self, layer: int, slot: int) -> None:
        if slot in self._free[layer] or any(p.slot == slot for p in self.clean[layer]):
            raise RuntimeError(f"[paged] layer {layer}: slot {slot} released twice or still clean")
        self._free[layer].append(slot)

    def pack(self, layer: int, slot: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Quantize one chunk's rotated K and V [T, H, D] (or [1, T, H, D]) into ``slot``."""
        self.pools[layer].pack(k, v, self.table(layer, [slot]))

    # ----------------------------------------------------------- clean list
    def append_clean(self, layer: int, page: CleanPage) -> None:
        """``_append_clean_page`` (common.py:110-114) over slots: keep the anchor and the last 7."""
        lst = self.clean[layer]
        lst.append(page)
        self._clean_version += 1
        if len(lst) > MAX_CLEAN:
            dropped = lst[1:len(lst) - (MAX_CLEAN - 1)]
            lst[:] = lst[:1] + lst[-(MAX_CLEAN - 1):]
            for p in dropped:
                self._free[layer].append(p.slot)

    def anchor_ku_out(self, layer: int) -> torch.Tensor | None:
        """[T, H*D] bf16 buffer for ``layer``'s normalized, un-rotated K while the current store pass's chunk
        is the anchor-to-be (the first chunk stored), else None.  The stored K is the ``ku`` the reference
        keeps for the anchor re-RoPE (common.py:83-88)."""
        if self._store is None or self.clean[layer]:
            return None
        if self.anchor_ku is None:
            self.anchor_ku = torch.empty((self.n_layers, self.T, self.n_heads, self.head_dim), dtype=torch.bfloat16,
                                         device=self.device)
        return self.anchor_ku[layer].view(self.T, self.n_heads * self.head_dim)

    def _working(self, layer: int, qf: int) -> list[CleanPage]:
        lst = self.clean[layer]
        _, n_work = anchor_and_working(len(lst), working_chunks(self.max_attn_frames, qf, self.npb))
        return lst[len(lst) - n_work:] if n_work else []

    def prepare_pass(self, p: Pass, height: int, width: int) -> None:
        """Rotate every layer's anchor K to this pass's ``rope_start`` (common.py:70-91) in one launch, unless
        its pages already hold that rotation.  All layers share one clean-list length and geometry."""
        key = (height, width, self._clean_version)
        if self._prepared is not None and self._prepared[0] is p and self._prepared[1] == key:
            return
        self._prepare_pass(p, height, width)
        self._prepared = (p, key)

    def _prepare_pass(self, p: Pass, height: int, width: int) -> None:
        if not self.clean[0]:
            return
        if any(len(c) != len(self.clean[0]) for c in self.clean):
            raise RuntimeError("[paged] the layers' clean lists differ in length")
        start = anchor_rope_start(p.csf, len(self._working(0, p.qf)), self.npb)
        if self._anchor_rot == (start, height, width):
            return
        if self.npb * height * width != self.T:
            raise ValueError(f"grid {self.npb}x{height}x{width} does not hold the chunk's {self.T} tokens")
        cos, sin = rope.cos_sin(self.npb, height, width, start, self.head_dim, device=self.device)
        anchors = tuple(c[0].slot for c in self.clean)
        key = ("anchors", anchors)
        table = self._tables.get(key)
        if table is None:
            ppl = self.pages_per_layer
            table = self.pool.page_table([L * ppl + pg for L, s in enumerate(anchors) for pg in self.slot_pages(s)])
            self._tables[key] = table
        self.pool.pack(self.anchor_ku.view(self.n_layers * self.T, self.n_heads, self.head_dim), None, table,
                       rope=(cos, sin), tiled=True)
        self._anchor_rot = (start, height, width)

    # ----------------------------------------------------------------- ticks
    def begin_tick(self, plan: TickPlan) -> TickPlan:
        if self._plan is not None:
            raise RuntimeError("[paged] the previous tick has not ended (end_tick / abort_tick)")
        if plan.act_ranks and (min(plan.act_ranks) < 0 or max(plan.act_ranks) >= self.rf_step):
            raise ValueError(f"[paged] active ranks {plan.act_ranks} outside 0..{self.rf_step - 1}")
        # slot tuples recur as the ring turns, but the cache is bounded anyway; it is only cleared between ticks,
        # where no kernel of this exchange's passes is still queued behind a stream the caller has not joined
        if len(self._tables) >= TABLE_CACHE_MAX:
            self._tables.clear()
        self._plan = plan
        return plan

    def begin_tick_at(self, tick: int, num_chunks: int) -> TickPlan:
        """Begin tick ``tick`` of a stream of ``num_chunks`` chunks with the reference's schedule."""
        return self.begin_tick(tick_plan(tick, self.rf_step, num_chunks, self.npb))

    def _require_plan(self) -> TickPlan:
        if self._plan is None:
            raise RuntimeError("[paged] no tick in progress (begin_tick)")
        return self._plan

    def store_pass(self) -> Pass:
        """The store rank's pass of this tick: chunk tick - rf_step with the one-chunk geometry."""
        plan = self._require_plan()
        if not plan.store_active:
            raise RuntimeError(f"[paged] the store rank is idle at tick {plan.tick}")
        if self._store is not None:
            raise RuntimeError("[paged] one store pass per tick")
        c = plan.tick - self.rf_step
        self._store = Pass("store", c, self.rf_step, c * self.npb, self.npb)
        return self._store

    def denoise_pass(self, rank: int) -> Pass:
        """Denoise rank ``rank``'s pass of this tick: chunk tick - rank with the tick's geometry."""
        plan = self._require_plan()
        if rank not in plan.act_ranks:
            raise RuntimeError(f"[paged] rank {rank} is idle at tick {plan.tick} (active {plan.act_ranks})")
        return Pass("denoise", plan.tick - rank, rank, plan.csf, plan.qf)

    def _own_slot(self, layer: int, p: Pass) -> int:
        held = self._live if p.kind == "store" else self._inflight[layer]
        key = layer if p.kind == "store" else p.rank
        slot = held.get(key)
        if slot is None:
            slot = held[key] = self.reserve(layer)
        return slot

    def context_slots(self, layer: int, p: Pass) -> tuple[list[int], int]:
        """(context slots in the reference's order, the pass's own slot) of ``layer``: store
        [anchor, working..., self] or denoise [anchor, working..., live, self, n > r ...]."""
        lst = self.clean[layer]
        geo = self._geometry
        if geo is None or geo[0] is not p or geo[1] != self._clean_version or len(lst) != geo[3]:
            n = len(lst)
            n_work = len(self._working(layer, p.qf)) if n else 0
            above = inflight_order(p.rank, self._plan.act_ranks)[1:] if p.kind == "denoise" else []
            geo = self._geometry = (p, self._clean_version, ([0] + list(range(n - n_work, n))) if n else [], n,
                                    above)
        aw = [lst[i].slot for i in geo[2]]
        if p.kind == "store":
            own = self._own_slot(layer, p)
            return aw + [own], own
        plan = self._plan
        slots = list(aw)
        if plan.store_active:
            live = self._live.get(layer)
            if live is None:
                raise RuntimeError(f"[paged] layer {layer}: the store pass has not published this layer "
                                   "(run the store pass first)")
            slots.append(live)
        above = geo[4]
        for n in above:
            if n not in self._inflight[layer]:
                raise RuntimeError(f"[paged] layer {layer}: rank {n} has not published this layer "
                                   "(run the denoise ranks from the highest down)")
        if len(slots) + 1 + len(above) > self.n_slots:
            raise RuntimeError(f"[paged] active_slots={len(slots) + 1 + len(above)} > {self.n_slots}")
        own = self._own_slot(layer, p)
        return slots + [own] + [self._inflight[layer][n] for n in above], own

    def layer_context(self, layer: int, p: Pass, height: int, width: int):
        """(pool, context table, own table, context keys) of ``layer`` for a block that packs its own K/V
        into the own table (QuantizedWanBlock.forward); the anchor is rotated for the pass first."""
        self.prepare_pass(p, height, width)
        slots, own = self.context_slots(layer, p)
        return self.pools[layer], self.table(layer, slots), self.table(layer, [own]), len(slots) * self.T

    def end_tick(self) -> None:
        """Promote the stored chunk into every layer's clean list (engine.py:433-503) and release the
        in-flight slots."""
        self._require_plan()
        if self._store is not None:
            if set(self._live) != set(range(self.n_layers)):
                raise RuntimeError("[paged] the store pass did not publish every layer")
            first = not self.clean[0]
            for L in range(self.n_layers):
                self.append_clean(L, CleanPage(cid=self._store.chunk, slot=self._live[L]))
            if first:
                self._anchor_rot = None
        for L in range(self.n_layers):
            for slot in self._inflight[L].values():
                self.release(L, slot)
            self._inflight[L] = {}
        self._live = {}
        self._store = None
        self._plan = None

    def reset(self) -> None:
        """Start a new stream: empty every layer's clean list and return every slot, as each run of the
        reference's tick loop starts from fresh clean lists (engine.py:294).  The anchor K buffer is kept
        for reuse."""
        if self._plan is not None:
            raise RuntimeError("[paged] a tick is in progress (end_tick / abort_tick first)")
        for L in range(self.n_layers):
            self.clean[L] = []
            self._free[L] = list(range(self.n_slots))
            self._inflight[L] = {}
        self._live = {}
        self._store = None
        self._anchor_rot = None
        self._clean_version += 1
        self._prepared = None
        self._geometry = None

    def abort_tick(self) -> None:
        """Return every slot the tick holds without promoting anything."""
        for L, slot in self._live.items():
            self.release(L, slot)
        for L in range(self.n_layers):
            for slot in self._inflight[L].values():
                self.release(L, slot)
            self._inflight[L] = {}
        self._live = {}
        self._store = None
        self._plan = None

    # ------------------------------------------------------------- closures
    def make_denoise_exch(self, rank: int):
        """Denoise-side exchange of rank ``rank`` (``_make_denoise_exch_paged``, paged.py:156-255): pack the
        rank's K/V into its slot, rotate the anchor, return the context descriptor."""
        p = self.denoise_pass(rank)

        def exch(*, layer_idx, roped_query, roped_key, unroped_key, value, current_start=None,
                 tokens_per_frame=None, post_patch_height, post_patch_width, dim=None, rope_num_heads=None,
                 num_frames_per_block=None):
            pool, ctx, own, n = self.layer_context(layer_idx, p, post_patch_height, post_patch_width)
            pool.pack(roped_key, value, own)
            kv = PagedKV(pool, ctx, n)
            return kv, kv

        return exch

    def make_store_exch(self):
        """Store-side exchange (``_make_store_exch_paged``, paged.py:257-310): the chunk's K/V go into its
        slot, which :meth:`end_tick` hands to the clean list; the first stored chunk keeps its
        un-rotated K for the anchor re-RoPE."""
        p = self.store_pass()

        def exch(*, layer_idx, roped_query, roped_key, unroped_key, value, current_start=None,
                 tokens_per_frame=None, post_patch_height, post_patch_width, dim=None, rope_num_heads=None,
                 num_frames_per_block=None):
            L = layer_idx
            pool, ctx, own, n = self.layer_context(L, p, post_patch_height, post_patch_width)
            pool.pack(roped_key, value, own)
            keep = self.anchor_ku_out(L)
            if keep is not None:
                if unroped_key is None:
                    raise RuntimeError(f"[paged] layer {L}: the anchor chunk needs its unroped_key")
                keep.copy_(unroped_key.reshape(self.T, -1))
            kv = PagedKV(pool, ctx, n)
            return kv, kv

        return exch
