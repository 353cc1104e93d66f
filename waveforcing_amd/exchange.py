"""Paged FP8 KV exchange on one GPU.

Restates the fixed-slot paged exchange of WaveRT
(wave_rt/denoiser/exchange/paged.py:156-310) and its context assembly
(common.py:45-114) over FP8 page pools:

* the clean list per layer is the anchor (the first clean chunk) plus the last
  7 clean chunks (``_append_clean_page``, common.py:110-114);
* a step's context is the anchor, re-RoPEd so that it sits right before the
  working set, then the working set (the last ``wmax_chunks`` clean chunks),
  then the chunk itself (``_anchor_working``, common.py:70-91, and the slot
  geometry of ``_make_denoise_exch_paged``, paged.py:161-190);
* the closures keep the reference's keyword signature (paged.py:191-205) and
  return the context for the attention backend.

The reference holds clean chunks as bf16 tensors and copies anchor, working set
and self into fixed slots of a bf16 slab every layer of every step
(paged.py:215-237).  Here each chunk is quantized into its pages once, when it
is produced, and a context is a page table over those pages: the copies
disappear.  Only the anchor's K is rewritten each step, because its rotation
depends on the working set's length: ``wf_fp8_kv_pack_rope`` rotates the kept
un-rotated anchor key (``ku``) and packs it in one pass.  The anchor's V is
packed once.

Pages: every layer has its own :class:`~waveforcing_amd.kv.Fp8PagePool` of
``n_slots`` chunk slots of ``frames_per_chunk`` pages (one latent frame per
page).  Slots move between a free list, the clean list and in-flight use
(the chunk being denoised or stored); promotion of a stored chunk to the
clean list hands over its slot, and the slot of a chunk that falls out of
the clean list returns to the free list.  With one GPU there are no peers, so
publishing is the pack into this GPU's own slot and there are no flags to wait
on (paged.py:120-154).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from . import rope
from .kv import Fp8PagePool, PagedKV, PageTable

MAX_CLEAN = 8  # anchor + the last 7 clean chunks (common.py:110-114)


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


@dataclass
class CleanPage:
    """One chunk of the clean list: its slot, chunk id and, for the anchor, the un-rotated K."""

    cid: int
    slot: int
    ku: torch.Tensor | None = None


class PagedExchange:
    """Per-layer FP8 page pools, the clean lists, and the exchange closures."""

    def __init__(self, n_layers: int, n_heads: int, tokens_per_frame: int, frames_per_chunk: int = 3,
                 max_attn_frames: int = 21, head_dim: int = 128, n_inflight: int = 2, device="cuda") -> None:
        self.n_layers = n_layers
        self.n_heads = n_heads
        self.head_dim = head_dim
        self.npb = frames_per_chunk
        self.page_tokens = tokens_per_frame
        self.T = tokens_per_frame * frames_per_chunk
        self.max_attn_frames = max_attn_frames
        self.device = torch.device(device)
        self.n_slots = MAX_CLEAN + n_inflight
        self.pools = [Fp8PagePool(self.n_slots * frames_per_chunk, n_heads, head_dim, tokens_per_frame, device)
                      for _ in range(n_layers)]
        self.clean: list[list[CleanPage]] = [[] for _ in range(n_layers)]
        self._free: list[list[int]] = [list(range(self.n_slots)) for _ in range(n_layers)]
        self._tables: dict = {}
        self._denoise_slots: dict[int, int] = {}  # layer -> slot of the chunk being denoised

    # ---------------------------------------------------------------- slots
    def slot_pages(self, slot: int) -> list[int]:
        return [slot * self.npb + f for f in range(self.npb)]

    def table(self, layer: int, slots: list[int]) -> PageTable:
        key = (layer, tuple(slots))
        t = self._tables.get(key)
        if t is None:
            if len(self._tables) >= 4096:  # slot tuples recur as the ring turns; bound the cache anyway
                self._tables.clear()
            pages = [p for s in slots for p in self.slot_pages(s)]
            t = self.pools[layer].page_table(pages)
            self._tables[key] = t
        return t

    def reserve(self, layer: int) -> int:
        """Take a free slot of ``layer`` for a chunk in flight."""
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
        if not lst and page.ku is None:
            raise RuntimeError(f"[paged] layer {layer}: the first clean chunk is the anchor and needs its "
                               "un-rotated key")
        lst.append(page)
        if len(lst) > MAX_CLEAN:
            dropped = lst[1:len(lst) - (MAX_CLEAN - 1)]
            lst[:] = lst[:1] + lst[-(MAX_CLEAN - 1):]
            for p in dropped:
                self._free[layer].append(p.slot)

    def _anchor_working(self, layer: int, chunk_start_frame: int, query_frames: int, height: int,
                        width: int) -> list[int]:
        """Slots of anchor + working set, with the anchor's K re-RoPEd in its pages (common.py:70-91)."""
        lst = self.clean[layer]
        if not lst:
            return []
        n_anchor, n_work = anchor_and_working(len(lst), working_chunks(self.max_attn_frames, query_frames,
                                                                       self.npb))
        anchor = lst[0]
        working = lst[len(lst) - n_work:] if n_work > 0 else []
        start = anchor_rope_start(chunk_start_frame, len(working), self.npb)
        if self.npb * height * width != self.T:
            raise ValueError(f"grid {self.npb}x{height}x{width} does not hold the chunk's {self.T} tokens")
        cos, sin = rope.cos_sin(self.npb, height, width, start, self.head_dim, device=self.device)
        pool = self.pools[layer]
        pool.pack(anchor.ku, None, self.table(layer, [anchor.slot]), rope=(cos, sin))
        return [anchor.slot] + [p.slot for p in working]

    def _context(self, layer: int, slots: list[int]) -> PagedKV:
        return PagedKV(self.pools[layer], self.table(layer, slots), len(slots) * self.T)

    # ------------------------------------------------------------- closures
    def make_denoise_exch(self, chunk_start_frame: int, query_frames: int | None = None):
        """Denoise-side exchange (paged.py:156-255): pack self, re-RoPE the anchor, return the context.

        Each layer's chunk goes into a slot reserved on the layer's first call;
        :meth:`finish_denoise` releases them after the forward.
        """
        qf = self.npb if query_frames is None else query_frames
        if self._denoise_slots:
            raise RuntimeError("[paged] the previous denoise step still holds slots; call finish_denoise() first")

        def exch(*, layer_idx, roped_query, roped_key, unroped_key, value, current_start=None,
                 tokens_per_frame=None, post_patch_height, post_patch_width, dim=None, rope_num_heads=None,
                 num_frames_per_block=None):
            L = layer_idx
            slot = self._denoise_slots.get(L)
            if slot is None:
                slot = self._denoise_slots[L] = self.reserve(L)
            self.pack(L, slot, roped_key, value)
            slots = self._anchor_working(L, chunk_start_frame, qf, post_patch_height, post_patch_width)
            if len(slots) + 1 > self.n_slots:
                raise RuntimeError(f"[paged] active_slots={len(slots) + 1} > {self.n_slots}")
            ctx = self._context(L, slots + [slot])
            return ctx, ctx

        return exch

    def layer_context(self, layer: int, chunk_start_frame: int, query_frames: int, height: int, width: int,
                      store_kv: dict | None = None):
        """(pool, context table, own table, context keys) of one layer for a block that packs its own
        K/V (QuantizedWanBlock.forward): the chunk's slot is reserved (a denoise step's, released by
        finish_denoise; or, with ``store_kv``, the stored chunk's, recorded for promote), the
        anchor re-RoPEd, and the context is anchor + working set + the chunk."""
        if store_kv is not None:
            if layer not in store_kv:
                store_kv[layer] = (self.reserve(layer), None)
            slot = store_kv[layer][0]
        else:
            if layer not in self._denoise_slots:
                self._denoise_slots[layer] = self.reserve(layer)
            slot = self._denoise_slots[layer]
        ctx_slots = self._anchor_working(layer, chunk_start_frame, query_frames, height, width)
        if len(ctx_slots) + 1 > self.n_slots:
            raise RuntimeError(f"[paged] active_slots={len(ctx_slots) + 1} > {self.n_slots}")
        return (self.pools[layer], self.table(layer, ctx_slots + [slot]), self.table(layer, [slot]),
                (len(ctx_slots) + 1) * self.T)

    def finish_denoise(self) -> None:
        for L, slot in self._denoise_slots.items():
            self.release(L, slot)
        self._denoise_slots = {}

    def abort_store(self, store_kv: dict) -> None:
        """Return the slots of a store pass that will not be promoted."""
        for L, (slot, _) in store_kv.items():
            self.release(L, slot)
        store_kv.clear()

    def make_store_exch(self, chunk: int, store_kv: dict):
        """Store-side exchange (paged.py:257-310): the chunk's clean K/V go into a reserved slot that
        :meth:`promote` hands to the clean list; ``store_kv[L]`` = (slot, unroped_key)."""

        def exch(*, layer_idx, roped_query, roped_key, unroped_key, value, current_start=None,
                 tokens_per_frame=None, post_patch_height, post_patch_width, dim=None, rope_num_heads=None,
                 num_frames_per_block=None):
            L = layer_idx
            if L in store_kv:
                slot = store_kv[L][0]
            else:
                slot = self.reserve(L)
            self.pack(L, slot, roped_key, value)
            slots = self._anchor_working(L, chunk * self.npb, self.npb, post_patch_height, post_patch_width)
            store_kv[L] = (slot, unroped_key)
            ctx = self._context(L, slots + [slot])
            return ctx, ctx

        return exch

    def promote(self, store_kv: dict, cid: int) -> None:
        """Append the stored chunk to every layer's clean list (engine.py:433-503).

        The first clean chunk of a layer becomes its anchor and keeps a copy
        of its un-rotated key (the broadcast of ``ku`` for cid 0,
        engine.py:433-480); later chunks keep only their pages.
        """
        for L, (slot, ku) in sorted(store_kv.items()):
            keep = None
            if not self.clean[L]:
                if ku is None:
                    raise RuntimeError(f"[paged] layer {L}: the anchor chunk needs its unroped_key")
                k = ku[0] if ku.dim() == 4 else ku
                if k.dim() == 2:  # [T, dim] rows of the block's K (QuantizedWanBlock unroped_k_out)
                    k = k.view(k.shape[0], self.n_heads, self.head_dim)
                keep = k.contiguous().clone()   # the caller may reuse its buffer
            self.append_clean(L, CleanPage(cid=cid, slot=slot, ku=keep))
        store_kv.clear()
