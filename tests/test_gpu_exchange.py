"""GPU parity of the single-GPU paged exchange over a whole wavefront.

Ticks 0..14 of an 11-chunk stream at rf_step 4 with a 21-frame window
(wave_rt/denoiser/engine.py:300-420): every pass of every tick calls its
exchange closure through the patched-forward route of
wave_rt/runtime/backend.py:87-157 -- ``set_exchange_fn(closure)``, then
``exchange_and_attend`` with the ``hip_fp8`` backend and profiling on.

A plain list model of the reference's contexts, holding bf16 tensors as the
reference does, builds each pass's K/V: store [anchor, working..., self]
(common.py:93-107), denoise [anchor, working..., live, self, in-flight
n > r ...] (paged.py:161-190), the anchor re-RoPEd by the oracle's table
rotation at ``csf - wflen - npb``.  Checked for every (pass, layer):

* the oracle's per-(token, head) quantize/dequantize of that context equals,
  bit for bit, the dequantized pages the closure hands to attention;
* the attention output equals the oracle's fp32 SDPA over that context within
  2e-2 max-abs (with the ``hip_fp8_qk`` backend, the oracle's quantized-QK
  attention over the context's codes, with ``hip_fp8_qkpv`` the oracle's
  fp8-PV attention over the K and V codes, beyond its rounding margin for
  weights within 2^-15 of an e4m3 rounding midpoint; same bar);
* ``prof_read()`` reports the context length as ``klen`` and positive
  exchange and attention times.

The steady-state denoise context of rank 0 is 8 chunks: anchor + 2 working
+ live + self + 3 in-flight.
"""

import pytest
import torch

from oracle import attention as oat
from oracle import block as ob
from oracle import kv as okv
from waveforcing_amd import backend
from waveforcing_amd import exchange as ex

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
NPB, HT, WD, H = 3, 8, 8, 2          # 3-frame chunks of 8 x 8 tokens per frame, 2 heads
T = NPB * HT * WD
WINDOW, RF, N_CHUNKS, LAYERS = 21, 4, 11, 2


def _kv(t, rank, layer):
    g = torch.Generator().manual_seed(100000 + 1000 * t + 10 * rank + layer)
    mk = lambda: torch.randn((1, T, H, 128), generator=g).to(torch.bfloat16)   # the workload's N(0, 1)
    return mk(), mk(), mk(), mk()          # q, roped K, un-rotated K, V


def _model_context(clean, live, inflight, plan, rank, layer, raw=False):
    """Dequantized K, V of the list model's context for a pass (rank RF = store); with ``raw`` the bf16 K and
    V before their FP8 round trip."""
    if rank == RF:
        csf, qf = (plan.tick - RF) * NPB, NPB
    else:
        csf, qf = plan.csf, plan.qf
    ks, vs = [], []
    if clean:
        _, n_w = ex.anchor_and_working(len(clean), ex.working_chunks(WINDOW, qf, NPB))
        working = clean[len(clean) - n_w:] if n_w else []
        ang = ob.rope_angles(NPB, HT, WD, ex.anchor_rope_start(csf, len(working), NPB))
        ks.append(ob.rope_apply_table(clean[0]["ku"][layer][0], torch.cos(ang).float(), torch.sin(ang).float()))
        vs.append(clean[0]["v"][layer][0])
        ks += [w["kr"][layer][0] for w in working]
        vs += [w["v"][layer][0] for w in working]
    if rank == RF:
        chunks = [live]
    else:
        chunks = ([live] if plan.store_active else []) + [inflight[n] for n in ex.inflight_order(rank, plan.act_ranks)]
    ks += [c["kr"][layer][0] for c in chunks]
    vs += [c["v"][layer][0] for c in chunks]
    if raw:
        return torch.cat(ks, 0), torch.cat(vs, 0)
    rt = lambda x: okv.dequantize_rows(*okv.quantize_rows(x))
    return rt(torch.cat(ks, 0)), rt(torch.cat(vs, 0))


@pytest.mark.parametrize("attn", ["hip_fp8", "hip_fp8_qk", "hip_fp8_qkpv"])
def test_wavefront_contexts_and_patched_attention_match_list_model(attn):
    x = ex.PagedExchange(n_layers=LAYERS, n_heads=H, tokens_per_frame=HT * WD, frames_per_chunk=NPB,
                         max_attn_frames=WINDOW, rf_step=RF, device=DEV)
    {"hip_fp8": backend.enable_hip_fp8, "hip_fp8_qk": backend.enable_hip_fp8_qk,
     "hip_fp8_qkpv": backend.enable_hip_fp8_qkpv}[attn]()
    clean = []
    longest = 0
    try:
        for t in range(N_CHUNKS + RF):
            plan = x.begin_tick_at(t, N_CHUNKS)
            live, inflight = None, {}
            order = ([RF] if plan.store_active else []) + sorted(plan.act_ranks, reverse=True)
            for rank in order:
                closure = x.make_store_exch() if rank == RF else x.make_denoise_exch(rank)
                seen = []

                def recording(**kw):
                    seen.append(closure(**kw))
                    return seen[-1]

                backend.set_exchange_fn(recording)
                entry = {"kr": [], "ku": [], "v": []}
                for layer in range(LAYERS):
                    q, kr, ku, v = _kv(t, rank, layer)
                    entry["kr"].append(kr)
                    entry["ku"].append(ku)
                    entry["v"].append(v)
                    if rank == RF:
                        live = entry
                    else:
                        inflight[rank] = entry
                    backend.prof_reset(True)
                    out = backend.exchange_and_attend(layer, q.to(DEV), kr.to(DEV), ku.to(DEV), v.to(DEV),
                                                      current_start=(t - rank) * NPB * HT * WD,
                                                      tokens_per_frame=HT * WD, post_patch_height=HT,
                                                      post_patch_width=WD, dim=H * 128, rope_num_heads=H,
                                                      num_frames_per_block=NPB)
                    attn_ms, exch_ms, klen = backend.prof_read()
                    ctx, ctx_v = seen[-1]
                    assert ctx_v is ctx
                    wk, wv = _model_context(clean, live, inflight, plan, rank, layer)
                    k, vv = ctx.pool.unpack(ctx.table, ctx.n_tokens)
                    assert ctx.shape == (1, wk.shape[0], H, 128) and klen == wk.shape[0]
                    assert torch.equal(k.cpu(), wk) and torch.equal(vv.cpu(), wv), f"tick {t} rank {rank} L{layer}"
                    assert attn_ms > 0 and exch_ms > 0
                    if attn == "hip_fp8":
                        ref, margin = oat.sdpa(q[0], wk, wv), 0.0
                    else:
                        rk, rv = _model_context(clean, live, inflight, plan, rank, layer, raw=True)
                        kc, ksc = okv.quantize_rows(rk)
                        ref, margin = (oat.sdpa_qk8(q[0], kc, ksc, wv), 0.0) if attn == "hip_fp8_qk" else \
                            oat.sdpa_qkpv8(q[0], kc, ksc, *okv.quantize_rows(rv), margin_eps=2.0 ** -15)
                    err = ((out[0].cpu().float() - ref).abs() - margin).max().item()
                    assert out.shape == q.shape and err <= 2e-2, f"tick {t} rank {rank} L{layer}: {err:.3e}"
                    longest = max(longest, wk.shape[0])
            backend.set_exchange_fn(None)
            x.end_tick()
            if plan.store_active:
                clean.append(live)
                if len(clean) > 8:
                    clean[:] = clean[:1] + clean[-7:]
            for layer in range(LAYERS):
                assert len(x.clean[layer]) == len(clean)
    finally:
        backend.set_exchange_fn(None)
        backend.prof_reset(False)
        backend._WAVE_STATE["attn"] = "torch_sdpa"
        backend._WAVE_STATE["fa_func"] = None
    torch.cuda.synchronize()
    assert longest == 8 * T     # anchor + 2 working + live + self + 3 in-flight
