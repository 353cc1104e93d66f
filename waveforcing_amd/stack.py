"""A stack of quantized Wan blocks over one chunk, with the paged FP8 exchange.

The block loop of one DiT forward for one chunk at one denoising step
(WaveBackend.forward_chunk, wave_rt/runtime/backend.py:456-490, whose
transformer runs ``for block in self.blocks``), each layer's self-attention
context coming from the paged exchange (waveforcing_amd.exchange): every block
packs its own K/V into its chunk's slot straight from the QKV projection
(wf_k_norm_rope_kv_pack) and attends to anchor + working set + that slot.

Only the blocks are on the quantized path: the DiT's patch embedding, time and
text embeddings and output head are not rebuilt here, so the caller hands in
the chunk's hidden states x [T, dim], its time modulation e [F, 6, dim] and
the text context.
"""

from __future__ import annotations

import torch

from . import rope
from .block import PRESETS, QuantizedWanBlock, apply_pending_residual, random_block_params
from .exchange import PagedExchange


class QuantizedWanStack:
    """``n_layers`` QuantizedWanBlocks sharing one PagedExchange (one FP8 page pool per layer)."""

    def __init__(self, blocks: list[QuantizedWanBlock], exchange: PagedExchange) -> None:
        if len(blocks) != exchange.n_layers:
            raise ValueError(f"{len(blocks)} blocks for an exchange of {exchange.n_layers} layers")
        self.blocks = blocks
        self.exchange = exchange
        # the layers run one after another: one set of activation buffers serves them all
        for b in blocks[1:]:
            b.share_workspace(blocks[0])
        # every layer's modulation table, so one add per chunk forms all the ``modulation + e``
        self._modulation = torch.stack([b.modulation[0] for b in blocks])   # [L, 6, dim]
        self.text_kv: list | None = None

    @classmethod
    def random(cls, preset: str = "1.3b", n_layers: int | None = None, seed: int = 0, device="cuda",
               tokens_per_frame: int = 1560, frames_per_chunk: int = 3, max_attn_frames: int = 24):
        """Seeded random-init blocks of a Wan preset (block.random_block_params, drawn on ``device``)."""
        cfg = PRESETS[preset]
        n = cfg["layers"] if n_layers is None else n_layers
        blocks = [QuantizedWanBlock(random_block_params(cfg["dim"], cfg["ffn_dim"], seed=seed + i, device=device),
                                    cfg["heads"], device) for i in range(n)]
        ex = PagedExchange(n, cfg["heads"], tokens_per_frame, frames_per_chunk, max_attn_frames, device=device)
        return cls(blocks, ex)

    def set_text(self, context: torch.Tensor) -> None:
        """Cross-attention K/V of the text context for every layer (once per request)."""
        self.text_kv = [blk.text_kv(context) for blk in self.blocks]

    def forward_chunk(self, x: torch.Tensor, e: torch.Tensor, chunk: int, height: int, width: int,
                      store: bool = False, query_frames: int | None = None) -> torch.Tensor:
        """Advance x [T, dim] bf16 in place through every layer for chunk ``chunk`` (latent frames
        chunk * npb ...).  A denoise step (store=False) releases the chunk's slots at the end; a store
        pass (store=True) keeps its K/V in their slots and adds them to every layer's clean list,
        the first such chunk becoming the anchor with its un-rotated K kept for re-RoPE.  On an error x
        is left partly updated and the chunk's slots are returned."""
        if self.text_kv is None:
            raise RuntimeError("set_text() first")
        ex = self.exchange
        npb = ex.npb
        # a store pass's context geometry is one chunk's (make_store_exch, paged.py:257-310)
        qf = npb if (store or query_frames is None) else query_frames
        csf = chunk * npb
        cos, sin = rope.cos_sin(npb, height, width, csf, ex.head_dim, device=x.device)
        store_kv: dict | None = {} if store else None
        es_all = self._modulation.unsqueeze(1) + e.unsqueeze(0)   # [L, F, 6, dim], one bf16 add
        pending = None
        try:
            for L, blk in enumerate(self.blocks):
                pool, ctx, own, n_ctx = ex.layer_context(L, csf, qf, height, width, store_kv)
                ku = None
                if store and not ex.clean[L]:
                    # the anchor-to-be (once per stream): keep its normalized, un-rotated K
                    ku = torch.empty_like(x)
                    store_kv[L] = (store_kv[L][0], ku)
                # each block's last gated residual runs fused into the next block's first LayerNorm
                x, pending = blk.forward(x, e, cos, sin, pool, ctx, own, n_ctx, self.text_kv[L], unroped_k_out=ku,
                                         es=es_all[L], pending=pending, defer_residual=True)
            apply_pending_residual(x, pending, x.shape[0] // e.shape[0])
        except BaseException:
            if store:
                ex.abort_store(store_kv)
            else:
                ex.finish_denoise()
            raise
        if store:
            ex.promote(store_kv, cid=chunk)
        else:
            ex.finish_denoise()
        return x
