"""The HIP path on the committed fixtures (tests/golden/): the same bars as
the other GPU parity tests -- codes, scales, int32 accumulators and int8 bf16
outputs bit-exact; GELU and e4m3 GEMM outputs within 1e-2 relative;
attention within 2e-2 of the fp32 reference (relative to max(1, |ref|), the
K/V being heavy-tailed); the two-layer toy block within relative L2 1e-2 and
max 5e-2 * max|x| after each layer."""

import os

import numpy as np
import pytest
import torch

from oracle import kv as okv
from waveforcing_amd import _lib, rope
from waveforcing_amd.backend import attn_paged_fp8
from waveforcing_amd.block import BlockParams, QuantizedWanBlock
from waveforcing_amd.fp8 import _quant_rows_i8, fp8_quant_pertensor, gemm_fp8_pertensor, gemm_i8
from waveforcing_amd.kv import Fp8PagePool, PagedKV

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
GOLD = os.path.join(os.path.dirname(__file__), "golden")


def load(name):
    return np.load(os.path.join(GOLD, name))


def bf(a):
    return torch.from_numpy(np.ascontiguousarray(a)).view(torch.bfloat16)


def rel(a, b):
    a, b = a.double(), b.double()
    return float((a - b).norm() / b.norm())


def test_kv_2pages_fixture():
    d = load("kv_2pages.npz")
    page, P = int(d["page_tokens"]), int(d["pool_pages"])
    k, v = bf(d["k_bits"]), bf(d["v_bits"])
    pool = Fp8PagePool(P, k.shape[1], 128, page, DEV)
    table = pool.page_table(d["table"].tolist())
    pool.pack(k.to(DEV), v.to(DEV), table)
    assert np.array_equal(pool.k_codes.cpu().numpy(), d["k_codes"])
    assert np.array_equal(pool.v_codes.cpu().numpy(), d["v_codes"])
    assert np.array_equal(pool.k_scales.cpu().numpy(), d["k_scales"])
    assert np.array_equal(pool.v_scales.cpu().numpy(), d["v_scales"])
    ko, vo = pool.unpack(table, k.shape[0])
    ids = d["table"].tolist()
    assert torch.equal(ko.cpu(), okv.unpack(ids, k.shape[0], page, torch.from_numpy(d["k_codes"]),
                                            torch.from_numpy(d["k_scales"])))
    assert torch.equal(vo.cpu(), okv.unpack(ids, v.shape[0], page, torch.from_numpy(d["v_codes"]),
                                            torch.from_numpy(d["v_scales"])))


def test_w8a8_small_fixture():
    d = load("w8a8_small.npz")
    x, w, b = bf(d["x_bits"]).to(DEV), bf(d["w_bits"]).to(DEV), bf(d["b_bits"]).to(DEV)
    qx, sx = _quant_rows_i8(x)
    qw, sw = _quant_rows_i8(w)
    assert np.array_equal(qx.cpu().numpy(), d["i8_qx"]) and np.array_equal(sx.cpu().numpy(), d["i8_sx"])
    assert np.array_equal(qw.cpu().numpy(), d["i8_qw"]) and np.array_equal(sw.cpu().numpy(), d["i8_sw"])
    acc = torch.empty(tuple(d["i8_acc"].shape), dtype=torch.int32, device=DEV)
    y = gemm_i8(qx, qw, sx, sw, b, acc_out=acc)
    assert np.array_equal(acc.cpu().numpy(), d["i8_acc"])
    assert torch.equal(y.cpu(), bf(d["i8_y_bits"]))
    yg = gemm_i8(qx, qw, sx, sw, b, gelu=True)
    assert rel(yg.cpu(), bf(d["i8_y_gelu_bits"])) < 1e-2
    wc, ws = fp8_quant_pertensor(w, _lib.FP8_TENSOR_WEIGHT)
    xc, xs = fp8_quant_pertensor(x, _lib.FP8_TENSOR_ACT)
    assert np.array_equal(wc.cpu().view(torch.uint8).numpy(), d["fp8_w_codes"])
    assert np.array_equal(ws.cpu().reshape(1).numpy(), d["fp8_w_scale"])
    assert np.array_equal(xc.cpu().view(torch.uint8).numpy(), d["fp8_x_codes"])
    assert torch.equal(xs.cpu().reshape(1), bf(d["fp8_x_scale_bits"]).float())
    y8 = gemm_fp8_pertensor(xc, wc, xs, ws, b)
    assert rel(y8.cpu(), bf(d["fp8_y_bits"])) < 1e-2


def test_attn_small_fixture():
    d = load("attn_small.npz")
    page, P = int(d["page_tokens"]), int(d["pool_pages"])
    q = bf(d["q_bits"])
    H, n_kv = q.shape[1], bf(d["k_bits"]).shape[0]
    pool = Fp8PagePool(P, H, 128, page, DEV)
    pool.k_codes.copy_(torch.from_numpy(d["k_codes"]))
    pool.v_codes.copy_(torch.from_numpy(d["v_codes"]))
    pool.k_scales.copy_(torch.from_numpy(d["k_scales"]))
    pool.v_scales.copy_(torch.from_numpy(d["v_scales"]))
    ctx = PagedKV(pool, pool.page_table(d["table"].tolist()), n_kv)
    out = attn_paged_fp8(q.to(DEV), ctx).cpu().float()
    ref = torch.from_numpy(d["out"])
    err = ((out - ref).abs() / ref.abs().clamp(min=1.0)).max().item()
    assert err <= 2e-2, err


def test_block_toy_fixture():
    d = load("block_toy.npz")
    c = {k[4:]: int(d[k]) for k in d.files if k.startswith("cfg_")}
    frames, h, w, heads = c["frames"], c["h"], c["w"], c["heads"]
    T, page, P = frames * h * w, h * w, int(d["pool_pages"])
    n_prior = c["prior_chunks"] * T
    start = c["prior_chunks"] * frames
    x = bf(d["x_bits"]).to(DEV).clone()
    context = bf(d["context_bits"]).to(DEV)
    cos, sin = rope.cos_sin(frames, h, w, start, device=DEV)
    names = BlockParams.__dataclass_fields__.keys()
    for layer in range(c["layers"]):
        params = BlockParams(**{n: bf(d[f"l{layer}_{n}_bits"]) for n in names})
        blk = QuantizedWanBlock(params, heads, DEV)
        pool = Fp8PagePool(P, heads, 128, page, DEV)
        prior_ids, own_ids = d[f"l{layer}_prior_ids"].tolist(), d[f"l{layer}_own_ids"].tolist()
        pool.pack(bf(d[f"l{layer}_prior_k_bits"]).to(DEV), bf(d[f"l{layer}_prior_v_bits"]).to(DEV),
                  pool.page_table(prior_ids))
        tk, tv = blk.text_kv(context)
        assert torch.equal(tk.cpu(), bf(d[f"l{layer}_text_k_bits"])) or \
            rel(tk.cpu(), bf(d[f"l{layer}_text_k_bits"])) < 1e-2
        blk.forward(x, bf(d[f"l{layer}_e_bits"]).to(DEV), cos, sin, pool, pool.page_table(prior_ids + own_ids),
                    pool.page_table(own_ids), n_prior + T, (tk, tv))
        ref = bf(d[f"l{layer}_out_bits"]).double()
        out = x.cpu().double()
        r = ((out - ref).norm() / ref.norm()).item()
        mx = (out - ref).abs().max().item()
        print(f"layer {layer}: rel L2 {r:.3e}, max abs {mx:.3e}")
        assert r <= 1e-2 and mx <= 5e-2 * ref.abs().max().item()
