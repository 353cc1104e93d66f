"""The oracle reproduces the committed fixtures (tests/golden/, written by
tests/golden/make_golden.py from the oracle): integer and byte results
exactly, float results within a few ulps (CPU float kernels may reorder
reductions between machines)."""

import os

import numpy as np
import torch

from oracle import attention as oat
from oracle import block as ob
from oracle import kv as okv
from oracle import linear as olin
from waveforcing_amd.block import BlockParams

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def load(name):
    return np.load(os.path.join(GOLD, name))


def bf(a):
    return torch.from_numpy(np.ascontiguousarray(a)).view(torch.bfloat16)


def rel(a, b):
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm().clamp(min=1e-30))


def test_kv_2pages_fixture():
    d = load("kv_2pages.npz")
    page, P = int(d["page_tokens"]), int(d["pool_pages"])
    table = d["table"].tolist()
    for name in ("k", "v"):
        x = bf(d[f"{name}_bits"])
        c, s = okv.new_pool(P, page, x.shape[1], x.shape[2])
        okv.pack(x, table, page, c, s)
        assert np.array_equal(c.numpy(), d[f"{name}_codes"]) and np.array_equal(s.numpy(), d[f"{name}_scales"])


def test_w8a8_small_fixture():
    d = load("w8a8_small.npz")
    x, w, b = bf(d["x_bits"]), bf(d["w_bits"]), bf(d["b_bits"])
    qx, sx = olin.i8_quant_rows(x)
    qw, sw = olin.i8_quant_rows(w)
    assert np.array_equal(qx.numpy(), d["i8_qx"]) and np.array_equal(sx.numpy(), d["i8_sx"])
    assert np.array_equal(qw.numpy(), d["i8_qw"]) and np.array_equal(sw.numpy(), d["i8_sw"])
    y, acc = olin.i8_gemm(qx, qw, sx, sw, b)
    assert np.array_equal(acc.numpy(), d["i8_acc"])
    assert torch.equal(y, bf(d["i8_y_bits"]))
    yg, _ = olin.i8_gemm(qx, qw, sx, sw, b, gelu=True)
    assert rel(yg.float(), bf(d["i8_y_gelu_bits"]).float()) < 1e-3
    wf, ws = olin.fp8_quant_weight(w)
    xf, xs = olin.fp8_quant_act(x)
    assert np.array_equal(wf.view(torch.uint8).numpy(), d["fp8_w_codes"])
    assert np.array_equal(ws.reshape(1).numpy(), d["fp8_w_scale"])
    assert np.array_equal(xf.view(torch.uint8).numpy(), d["fp8_x_codes"])
    assert torch.equal(xs.reshape(1), bf(d["fp8_x_scale_bits"]))
    y8 = olin.fp8_linear(x, wf, ws, b)
    assert rel(y8.float(), bf(d["fp8_y_bits"]).float()) < 1e-3


def test_attn_small_fixture():
    d = load("attn_small.npz")
    page, P = int(d["page_tokens"]), int(d["pool_pages"])
    table = d["table"].tolist()
    q, k, v = bf(d["q_bits"]), bf(d["k_bits"]), bf(d["v_bits"])
    kp = okv.new_pool(P, page, k.shape[1], 128)
    vp = okv.new_pool(P, page, v.shape[1], 128)
    okv.pack(k, table, page, *kp)
    okv.pack(v, table, page, *vp)
    assert np.array_equal(kp[0].numpy(), d["k_codes"]) and np.array_equal(vp[1].numpy(), d["v_scales"])
    out = oat.paged_fp8(q, kp, vp, table, k.shape[0], page)
    assert rel(out, torch.from_numpy(d["out"])) < 1e-5


def toy_params(d, layer):
    names = BlockParams.__dataclass_fields__.keys()
    return BlockParams(**{n: bf(d[f"l{layer}_{n}_bits"]) for n in names})


def test_block_toy_fixture():
    d = load("block_toy.npz")
    c = {k[4:]: int(d[k]) for k in d.files if k.startswith("cfg_")}
    frames, h, w, heads = c["frames"], c["h"], c["w"], c["heads"]
    T, page, P = frames * h * w, h * w, int(d["pool_pages"])
    x = bf(d["x_bits"])
    context = bf(d["context_bits"])
    n_prior = c["prior_chunks"] * T
    for layer in range(c["layers"]):
        p = toy_params(d, layer)
        prior_ids, own_ids = d[f"l{layer}_prior_ids"].tolist(), d[f"l{layer}_own_ids"].tolist()
        pk = okv.new_pool(P, page, heads, 128)
        pv = okv.new_pool(P, page, heads, 128)
        okv.pack(bf(d[f"l{layer}_prior_k_bits"]), prior_ids, page, *pk)
        okv.pack(bf(d[f"l{layer}_prior_v_bits"]), prior_ids, page, *pv)
        tk, tv = ob.text_kv(p, context, heads)
        assert torch.equal(tk, bf(d[f"l{layer}_text_k_bits"]))
        x = ob.block_forward(p, x, bf(d[f"l{layer}_e_bits"]), (frames, h, w), c["prior_chunks"] * frames, pk, pv,
                             prior_ids + own_ids, own_ids, n_prior + T, page, tk, tv, heads)
        assert rel(x.float(), bf(d[f"l{layer}_out_bits"]).float()) < 1e-3
