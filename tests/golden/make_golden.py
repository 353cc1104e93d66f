"""Write the small golden fixtures under tests/golden/ from the CPU oracle.

Run from the repository root:  python tests/golden/make_golden.py

Fixtures (numpy .npz, no pickles):
  e4m3_tables.npz  enc_bf16[65536] u8: torch's e4m3fn cast of every bf16 bit
                   pattern; dec[256] f32: torch's decode of every code.
  kv_small.npz     a ragged 40-token, 2-head, head_dim-128 K/V pair packed into
                   a 5-page pool of 16-token pages through a shuffled page
                   table; inputs as bf16 bit patterns, pool codes and scales.
  kv_2pages.npz    K/V [2 x 1560, 2, 128] (heavy-tailed) packed into 1560-token
                   pages 3 and 1 of a 4-page pool.
  w8a8_small.npz   x [64, 256] (1 % outlier channels) . W [192, 256]^T + bias:
                   the int8 scheme (codes, scales, int32 acc, bf16 out, bf16
                   out with GELU-tanh) and the reference's per-tensor e4m3
                   linear (codes, scales, bf16 out of torch._scaled_mm).
  attn_small.npz   128 queries x 2 heads over 3 x 256 keys packed to FP8 in
                   256-token pages [4, 1, 3] of a 5-page pool; fp32 output.
  block_toy.npz    two Wan blocks (dim 256, 2 heads, FFN 512) in sequence on a
                   3 x 8 x 8 chunk with one prior chunk of FP8 context per
                   layer and 16 text tokens; every parameter, input and the
                   output after each layer.
bf16 tensors are stored as int16 bit patterns.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import attention as oat  # noqa: E402
from oracle import block as ob  # noqa: E402
from oracle import fp8 as ofp8  # noqa: E402
from oracle import kv as okv  # noqa: E402
from oracle import linear as olin  # noqa: E402
from waveforcing_amd import inputs  # noqa: E402
from waveforcing_amd.block import random_block_params  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def e4m3_tables() -> None:
    allbf = ofp8.all_bf16_as_f32()
    enc = ofp8.encode(allbf).numpy().copy()
    dec = ofp8.decode(torch.arange(256, dtype=torch.int32).to(torch.uint8)).numpy().copy()
    np.savez(os.path.join(OUT, "e4m3_tables.npz"), enc_bf16=enc, dec=dec)


def kv_small() -> None:
    T, H, D, page, pool_pages = 40, 2, 128, 16, 5
    k = inputs.heavy_tailed_kv(T, H, D, seed=11)
    v = inputs.heavy_tailed_kv(T, H, D, seed=12)
    # A few exact-tie and extreme rows: zeros, a single spike, values that
    # quantize to exact e4m3 midpoints.
    k[0] = 0
    k[1, 0] = 0
    k[1, 0, 5] = 3.0
    v[2, 1] = torch.linspace(-448, 448, D).to(torch.bfloat16)
    table = [3, 0, 4]
    kc, ks = okv.new_pool(pool_pages, page, H, D)
    vc, vs = okv.new_pool(pool_pages, page, H, D)
    okv.pack(k, table, page, kc, ks)
    okv.pack(v, table, page, vc, vs)
    np.savez(
        os.path.join(OUT, "kv_small.npz"),
        k_bits=k.view(torch.int16).numpy(), v_bits=v.view(torch.int16).numpy(),
        table=np.array(table, dtype=np.int32), page_tokens=np.int32(page), pool_pages=np.int32(pool_pages),
        k_codes=kc.numpy(), k_scales=ks.numpy(), v_codes=vc.numpy(), v_scales=vs.numpy(),
    )


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy()


def kv_2pages() -> None:
    T, H, D, page, pool_pages = 2 * 1560, 2, 128, 1560, 4
    k = inputs.heavy_tailed_kv(T, H, D, seed=21)
    v = inputs.heavy_tailed_kv(T, H, D, seed=22)
    table = [3, 1]
    kc, ks = okv.new_pool(pool_pages, page, H, D)
    vc, vs = okv.new_pool(pool_pages, page, H, D)
    okv.pack(k, table, page, kc, ks)
    okv.pack(v, table, page, vc, vs)
    np.savez_compressed(
        os.path.join(OUT, "kv_2pages.npz"), k_bits=bits(k), v_bits=bits(v), table=np.array(table, dtype=np.int32),
        page_tokens=np.int32(page), pool_pages=np.int32(pool_pages),
        k_codes=kc.numpy(), k_scales=ks.numpy(), v_codes=vc.numpy(), v_scales=vs.numpy(),
    )


def w8a8_small() -> None:
    M, K, N = 64, 256, 192
    x = inputs.outlier_activations(M, K, seed=61, chan_seed=62)
    w, b = inputs.linear_weights(N, K, w_seed=63, b_seed=64)
    qx, sx = olin.i8_quant_rows(x)
    qw, sw = olin.i8_quant_rows(w)
    y, acc = olin.i8_gemm(qx, qw, sx, sw, b)
    y_gelu, _ = olin.i8_gemm(qx, qw, sx, sw, b, gelu=True)
    wf, wscale = olin.fp8_quant_weight(w)
    xf, xscale = olin.fp8_quant_act(x)
    y_fp8 = olin.fp8_linear(x, wf, wscale, b)
    np.savez(
        os.path.join(OUT, "w8a8_small.npz"), x_bits=bits(x), w_bits=bits(w), b_bits=bits(b),
        i8_qx=qx.numpy(), i8_sx=sx.numpy(), i8_qw=qw.numpy(), i8_sw=sw.numpy(), i8_acc=acc.numpy(),
        i8_y_bits=bits(y), i8_y_gelu_bits=bits(y_gelu),
        fp8_x_codes=xf.view(torch.uint8).numpy(), fp8_x_scale_bits=bits(xscale.reshape(1)),
        fp8_w_codes=wf.view(torch.uint8).numpy(), fp8_w_scale=wscale.reshape(1).numpy(), fp8_y_bits=bits(y_fp8),
    )


def attn_small() -> None:
    Lq, H, D, page, pool_pages = 128, 2, 128, 256, 5
    n_kv = 3 * page
    g = torch.Generator().manual_seed(71)
    q = torch.randn((Lq, H, D), generator=g).to(torch.bfloat16)
    k = inputs.heavy_tailed_kv(n_kv, H, D, seed=72)
    v = inputs.heavy_tailed_kv(n_kv, H, D, seed=73)
    table = [4, 1, 3]
    kp = okv.new_pool(pool_pages, page, H, D)
    vp = okv.new_pool(pool_pages, page, H, D)
    okv.pack(k, table, page, *kp)
    okv.pack(v, table, page, *vp)
    out = oat.paged_fp8(q, kp, vp, table, n_kv, page)
    np.savez(
        os.path.join(OUT, "attn_small.npz"), q_bits=bits(q), k_bits=bits(k), v_bits=bits(v),
        table=np.array(table, dtype=np.int32), page_tokens=np.int32(page), pool_pages=np.int32(pool_pages),
        k_codes=kp[0].numpy(), k_scales=kp[1].numpy(), v_codes=vp[0].numpy(), v_scales=vp[1].numpy(),
        out=out.numpy(),
    )


BLOCK_TOY = dict(dim=256, heads=2, ffn=512, frames=3, h=8, w=8, prior_chunks=1, text_len=16, layers=2)


def block_toy() -> None:
    c = BLOCK_TOY
    dim, heads, ffn = c["dim"], c["heads"], c["ffn"]
    frames, h, w = c["frames"], c["h"], c["w"]
    T, page = frames * h * w, h * w
    g = torch.Generator().manual_seed(81)
    x = torch.randn((T, dim), generator=g).to(torch.bfloat16)
    context = torch.randn((c["text_len"], dim), generator=g).to(torch.bfloat16)
    n_prior = c["prior_chunks"] * T
    pages_prior = c["prior_chunks"] * frames
    P = pages_prior + frames + 1
    start_frame = c["prior_chunks"] * frames
    arrays = {"x_bits": bits(x), "context_bits": bits(context)}
    for layer in range(c["layers"]):
        params = random_block_params(dim, ffn, seed=90 + layer)
        e = (torch.randn((frames, 6, dim), generator=g) * 0.1).to(torch.bfloat16)
        prior_k = torch.randn((n_prior, heads, 128), generator=g).to(torch.bfloat16)
        prior_v = torch.randn((n_prior, heads, 128), generator=g).to(torch.bfloat16)
        ids = torch.randperm(P, generator=g).tolist()
        prior_ids, own_ids = ids[:pages_prior], ids[pages_prior:pages_prior + frames]
        pk = okv.new_pool(P, page, heads, 128)
        pv = okv.new_pool(P, page, heads, 128)
        okv.pack(prior_k, prior_ids, page, *pk)
        okv.pack(prior_v, prior_ids, page, *pv)
        tk, tv = ob.text_kv(params, context, heads)
        x = ob.block_forward(params, x, e, (frames, h, w), start_frame, pk, pv, prior_ids + own_ids, own_ids,
                             n_prior + T, page, tk, tv, heads)
        for name, val in vars(params).items():
            arrays[f"l{layer}_{name}_bits"] = bits(val)
        arrays.update({
            f"l{layer}_e_bits": bits(e), f"l{layer}_prior_k_bits": bits(prior_k),
            f"l{layer}_prior_v_bits": bits(prior_v),
            f"l{layer}_prior_ids": np.array(prior_ids, dtype=np.int32),
            f"l{layer}_own_ids": np.array(own_ids, dtype=np.int32),
            f"l{layer}_text_k_bits": bits(tk), f"l{layer}_out_bits": bits(x),
        })
    arrays["pool_pages"] = np.int32(P)
    arrays.update({f"cfg_{k}": np.int32(v) for k, v in c.items()})
    np.savez_compressed(os.path.join(OUT, "block_toy.npz"), **arrays)


if __name__ == "__main__":
    e4m3_tables()
    kv_small()
    kv_2pages()
    w8a8_small()
    attn_small()
    block_toy()
    for f in sorted(os.listdir(OUT)):
        print(f, os.path.getsize(os.path.join(OUT, f)))
