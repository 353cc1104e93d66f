"""GPU parity of the single-GPU paged exchange over several chunks.

A plain list model of the reference's clean list and context assembly
(wave_rt/denoiser/exchange/common.py:70-114, paged.py:156-310), holding bf16
tensors as the reference does, builds each step's context as anchor
(re-RoPEd by the oracle's table rotation at ``csf - wflen - npb``) + working
set + self.  The oracle's per-(token, head) quantize/dequantize of that
context must equal, bit for bit, the dequantized pages the exchange hands to
attention.  The store passes promote chunks 0..9, so the clean list wraps
(anchor + last 7) and slots are recycled.
"""

import pytest
import torch

from oracle import block as ob
from oracle import kv as okv
from waveforcing_amd import exchange as ex

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
NPB, HT, WD, H = 3, 8, 8, 2          # 3-frame chunks of 8 x 8 tokens per frame, 2 heads
T = NPB * HT * WD
WINDOW = 18                          # 18-frame attention window: 4 working chunks for one query chunk


def _chunk(seed):
    g = torch.Generator().manual_seed(seed)
    mk = lambda: (torch.randn((1, T, H, 128), generator=g) * 2).to(torch.bfloat16)
    return mk(), mk(), mk()          # roped K, un-rotated K, V


def _oracle_context(model, csf, qf, kr, v):
    """model: list of dicts(kr, ku, v) (anchor first) -> dequantized K, V of the context."""
    ks, vs = [], []
    if model:
        n_a, n_w = ex.anchor_and_working(len(model), ex.working_chunks(WINDOW, qf, NPB))
        working = model[len(model) - n_w:] if n_w else []
        start = csf - len(working) * NPB - NPB
        ang = ob.rope_angles(NPB, HT, WD, start)
        ak = ob.rope_apply_table(model[0]["ku"][0], torch.cos(ang).float(), torch.sin(ang).float())
        ks += [ak] + [w["kr"][0] for w in working]
        vs += [model[0]["v"][0]] + [w["v"][0] for w in working]
    ks.append(kr[0])
    vs.append(v[0])
    rt = lambda x: okv.dequantize_rows(*okv.quantize_rows(x))
    return rt(torch.cat(ks, 0)), rt(torch.cat(vs, 0))


def _check(ctx_pair, want):
    ctx, ctx_v = ctx_pair
    assert ctx_v is ctx
    k, v = ctx.pool.unpack(ctx.table, ctx.n_tokens)
    assert ctx.shape == (1, want[0].shape[0], H, 128)
    assert torch.equal(k.cpu(), want[0]) and torch.equal(v.cpu(), want[1])


def _call(exch, layer, kr, ku, v):
    return exch(layer_idx=layer, roped_query=None, roped_key=kr.to(DEV), unroped_key=ku.to(DEV), value=v.to(DEV),
                current_start=0, tokens_per_frame=HT * WD, post_patch_height=HT, post_patch_width=WD, dim=H * 128,
                rope_num_heads=H, num_frames_per_block=NPB)


def test_store_and_denoise_contexts_match_list_model():
    L = 2
    x = ex.PagedExchange(n_layers=L, n_heads=H, tokens_per_frame=HT * WD, frames_per_chunk=NPB,
                         max_attn_frames=WINDOW, device=DEV)
    model = [[] for _ in range(L)]
    for c in range(10):
        # denoise step for chunk c + 1 against the clean list of chunks < c
        exch = x.make_denoise_exch((c + 1) * NPB)
        for layer in range(L):
            kr, ku, v = _chunk(1000 * c + 10 * layer + 1)
            _check(_call(exch, layer, kr, ku, v), _oracle_context(model[layer], (c + 1) * NPB, NPB, kr, v))
        x.finish_denoise()
        # store pass for chunk c, then promotion into the clean list
        store_kv = {}
        exch = x.make_store_exch(c, store_kv)
        for layer in range(L):
            kr, ku, v = _chunk(1000 * c + 10 * layer)
            _check(_call(exch, layer, kr, ku, v), _oracle_context(model[layer], c * NPB, NPB, kr, v))
            page = dict(kr=kr, ku=ku, v=v)
            model[layer].append(page)
            if len(model[layer]) > 8:
                model[layer][:] = model[layer][:1] + model[layer][-7:]
        x.promote(store_kv, cid=c)
        for layer in range(L):
            assert len(x.clean[layer]) == len(model[layer])
    torch.cuda.synchronize()
