"""A stack of quantized Wan blocks over the wavefront's chunks, with the paged FP8 exchange.

The block loop of one DiT forward for one chunk at one denoising step
(WaveBackend.forward_chunk, wave_rt/runtime/backend.py:456-490, whose
transformer runs ``for block in self.blocks``), each layer's self-attention
context coming from the paged exchange (waveforcing_amd.exchange): every block
packs its own K/V into its chunk's slot straight from the QKV projection
(wf_qk_norm_rope_kv_pack) and attends to the context the exchange lays out
for the pass (anchor, working set, live and in-flight chunks).

A tick of the wavefront (wave_rt/denoiser/engine.py:300-420) runs the store
rank's pass and every active denoise rank's pass on this GPU
(:meth:`QuantizedWanStack.tick`): the store pass first, then the denoise
ranks, either one after another or, with ``concurrent=True``, as a layer
wavefront on one HIP stream per rank.  Rank r's layer L needs only layer L of
the ranks above it (their in-flight chunks), the dependency the reference's
per-layer flag waits express between GPUs (paged.py:147-154), so on one GPU
each rank's stream waits for an event the next rank up records after its
layer L; the ranks' kernels then fill the CUs and launch gaps a single pass
leaves idle.  Every rank brings its own activation buffers, and all of them
share the anchor rotation of the tick's denoise geometry.  The stack works on hidden states:
the DiT's embeddings and output head around it live in
waveforcing_amd.dit, so the caller hands in each pass's hidden states
x [T, dim], its time modulation e [F, 6, dim] and the text context.
"""

from __future__ import annotations

import torch

from . import rope
from .block import PRESETS, QuantizedWanBlock, apply_pending_residual, random_block_params
from .exchange import Pass, PagedExchange, TickPlan


class QuantizedWanStack:
    """``n_layers`` QuantizedWanBlocks sharing one PagedExchange (one FP8 page pool for every layer)."""

    def __init__(self, blocks: list[QuantizedWanBlock], exchange: PagedExchange) -> None:
        if len(blocks) != exchange.n_layers:
            raise ValueError(f"{len(blocks)} blocks for an exchange of {exchange.n_layers} layers")
        self.blocks = blocks
        self.exchange = exchange
        # the layers run one after another: one set of activation buffers serves them all
        for b in blocks[1:]:
            b.share_workspace(blocks[0])
        # every layer's modulation table, so one add per pass forms all the ``modulation + e``
        self._modulation = torch.stack([b.modulation[0] for b in blocks])   # [L, 6, dim]
        self.text_kv: list | None = None
        # the layer wavefront's streams, per-layer events and per-pass activation buffers (created on first use)
        self._streams: list = []
        self._events: list = []
        self._pass_ws: dict = {}

    @classmethod
    def random(cls, preset: str = "1.3b", n_layers: int | None = None, seed: int = 0, device="cuda",
               tokens_per_frame: int = 1560, frames_per_chunk: int = 3, max_attn_frames: int = 21,
               rf_step: int = 4):
        """Seeded random-init blocks of a Wan preset (block.random_block_params, drawn on ``device``)."""
        cfg = PRESETS[preset]
        n = cfg["layers"] if n_layers is None else n_layers
        blocks = [QuantizedWanBlock(random_block_params(cfg["dim"], cfg["ffn_dim"], seed=seed + i, device=device),
                                    cfg["heads"], device) for i in range(n)]
        ex = PagedExchange(n, cfg["heads"], tokens_per_frame, frames_per_chunk, max_attn_frames, rf_step=rf_step,
                           device=device)
        return cls(blocks, ex)

    def set_text(self, context: torch.Tensor) -> None:
        """Cross-attention K/V of the text context for every layer (once per request)."""
        self.text_kv = [blk.text_kv(context) for blk in self.blocks]

    def run_pass(self, x: torch.Tensor, e: torch.Tensor, p: Pass, height: int, width: int,
                 kv_only_last: bool = False) -> torch.Tensor | None:
        """Advance x [T, dim] bf16 in place through every layer as pass ``p`` of the current tick.  With
        ``kv_only_last`` (a store pass whose output is dropped) the last layer stops once its K/V are
        published: every page the pass writes is the same, x is left mid-layer and None is returned."""
        if self.text_kv is None:
            raise RuntimeError("set_text() first")
        if kv_only_last and p.kind != "store":
            raise ValueError("only a store pass can skip its last layer's output")
        ex = self.exchange
        cos, sin = rope.cos_sin(ex.npb, height, width, p.chunk * ex.npb, ex.head_dim, device=x.device)
        ex.prepare_pass(p, height, width)
        es_all = self._modulation.unsqueeze(1) + e.unsqueeze(0)   # [L, F, 6, dim], one bf16 add
        pending = None
        last = len(self.blocks) - 1
        for L, blk in enumerate(self.blocks):
            pool, ctx, own, n_ctx = ex.layer_context(L, p, height, width)
            ku = ex.anchor_ku_out(L) if p.kind == "store" else None
            # each block's last gated residual runs fused into the next block's first LayerNorm
            x, pending = blk.forward(x, e, cos, sin, pool, ctx, own, n_ctx, self.text_kv[L], unroped_k_out=ku,
                                     es=es_all[L], pending=pending, defer_residual=True,
                                     kv_only=kv_only_last and L == last)
        if kv_only_last:
            return None
        apply_pending_residual(x, pending, x.shape[0] // e.shape[0])
        return x

    # -- concurrent denoise passes
    def side_streams(self, n: int) -> list:
        """n HIP streams of this stack's device (default priority), created once and reused."""
        dev = self.blocks[0].device
        while len(self._streams) < n:
            self._streams.append(torch.cuda.Stream(device=dev))
        return self._streams[:n]

    def pass_workspaces(self, n: int, T: int) -> list:
        """Activation buffers for n concurrent passes of T tokens (created once per (slot, T))."""
        out = []
        for i in range(n):
            ws = self._pass_ws.get((i, T))
            if ws is None:
                ws = self._pass_ws[(i, T)] = self.blocks[0].new_workspace(T)
            out.append(ws)
        return out

    def run_wavefront(self, items: list, height: int, width: int, pre=None, post=None) -> None:
        """Advance each (x, e, pass) of ``items`` -- denoise passes of the current tick, ordered from the highest
        rank down -- in place through every layer, pass i on its own stream, as a wavefront over the layers: pass
        i's layer L waits for pass i - 1's layer L.  The anchor rotation of their common geometry, the RoPE
        tables and the modulation sums are prepared on the current stream first; ``pre(i)`` / ``post(i)``, if
        given, enqueue work of pass i on its stream before its first / after its last layer.  Returns with the
        current stream waiting for every pass."""
        if self.text_kv is None:
            raise RuntimeError("set_text() first")
        passes = [p for _, _, p in items]
        if any(p.kind != "denoise" for p in passes) or len({(p.csf, p.qf) for p in passes}) > 1:
            raise ValueError("a wavefront runs the denoise passes of one tick (one context geometry)")
        ranks = [p.rank for p in passes]
        if ranks != sorted(ranks, reverse=True) or len(set(ranks)) != len(ranks):
            raise ValueError(f"wavefront passes must run from the highest rank down, got ranks {ranks}")
        ex = self.exchange
        n = len(items)
        dev = self.blocks[0].device
        T = items[0][0].shape[0]
        ex.prepare_pass(passes[0], height, width)
        wss = self.pass_workspaces(n, T)
        state = []
        for x, e, p in items:
            cos, sin = rope.cos_sin(ex.npb, height, width, p.chunk * ex.npb, ex.head_dim, device=x.device)
            state.append([x, None, cos, sin, self._modulation.unsqueeze(1) + e.unsqueeze(0)])
        evs = self._events
        while len(evs) < n:
            evs.append([torch.cuda.Event() for _ in self.blocks])
        # every page table the passes read is built here, on the current stream, before the streams fork (in the
        # loop's order, so each rank's in-flight slot is taken after the ranks above it): the caching allocator
        # then ties them to the current stream, which waits for every side stream before it goes on
        ctxs = [[ex.layer_context(L, p, height, width) for p in passes] for L in range(len(self.blocks))]
        cur = torch.cuda.current_stream(dev)
        streams = self.side_streams(n)
        try:
            for i, st in enumerate(streams):
                st.wait_stream(cur)
                if pre is not None:
                    with torch.cuda.stream(st):
                        pre(i)
            for L, blk in enumerate(self.blocks):
                for i, (_, e, p) in enumerate(items):
                    st = streams[i]
                    with torch.cuda.stream(st):
                        if i > 0:
                            st.wait_event(evs[i - 1][L])
                        x, pending, cos, sin, es_all = state[i]
                        pool, ctx, own, n_ctx = ctxs[L][i]
                        x, pending = blk.forward(x, e, cos, sin, pool, ctx, own, n_ctx, self.text_kv[L],
                                                 es=es_all[L], pending=pending, defer_residual=True, ws=wss[i])
                        state[i][0], state[i][1] = x, pending
                        if i + 1 < n:
                            evs[i][L].record(st)
            for i, (x, e, p) in enumerate(items):
                with torch.cuda.stream(streams[i]):
                    apply_pending_residual(state[i][0], state[i][1], x.shape[0] // e.shape[0])
                    if post is not None:
                        post(i)
        finally:
            # whatever was enqueued completes before the current stream goes on (and before the tables above,
            # allocated on it, can be reused)
            for st in streams:
                cur.wait_stream(st)

    def tick(self, plan: TickPlan, inputs: dict, height: int, width: int, concurrent: bool = False) -> TickPlan:
        """One wavefront tick on this GPU: ``inputs`` maps "store" (when the store rank is active) and each
        active denoise rank to its (x, e); the store pass runs first, then the ranks from the highest down,
        each x advanced in place, one after another or (``concurrent``) as a layer wavefront on one stream
        per rank (bit-identical results); the stored chunk joins the clean lists at the end.  On an error
        the tick's slots are returned and nothing is promoted."""
        ex = self.exchange
        ex.begin_tick(plan)
        try:
            if plan.store_active:
                self.run_pass(*inputs["store"], ex.store_pass(), height, width)
            ranks = sorted(plan.act_ranks, reverse=True)
            if concurrent and len(ranks) > 1:
                self.run_wavefront([(*inputs[r], ex.denoise_pass(r)) for r in ranks], height, width)
            else:
                for r in ranks:
                    self.run_pass(*inputs[r], ex.denoise_pass(r), height, width)
        except BaseException:
            ex.abort_tick()
            raise
        ex.end_tick()
        return plan

    def forward_chunk(self, x: torch.Tensor, e: torch.Tensor, chunk: int, height: int, width: int,
                      store: bool = False) -> torch.Tensor:
        """One chunk alone as a tick of its own: a store pass (the chunk joins the clean lists) or a
        denoise pass of rank 0 with no live or other in-flight chunk."""
        ex = self.exchange
        npb = ex.npb
        if store:
            plan = TickPlan(chunk + ex.rf_step, [], True, 0, 0)
            self.tick(plan, {"store": (x, e)}, height, width)
        else:
            plan = TickPlan(chunk, [0], False, chunk * npb, npb)
            self.tick(plan, {0: (x, e)}, height, width)
        return x
