"""GPU parity of the FP8 codec and the paged KV pack / gather-dequant kernels
against the CPU oracle (bit-exact codes, scales and bf16 outputs)."""

import os

import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle import kv as okv
from waveforcing_amd import inputs
from waveforcing_amd.kv import Fp8PagePool, PageTable, fp8_decode, fp8_encode

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
GOLD = os.path.join(os.path.dirname(__file__), "golden", "kv_small.npz")


def _pool_to_cpu(pool):
    return (pool.k_codes.cpu(), pool.k_scales.cpu(), pool.v_codes.cpu(), pool.v_scales.cpu())


def test_encode_all_bf16_values():
    x = ofp8.all_bf16_as_f32()
    got = fp8_encode(x.to(DEV)).cpu()
    assert torch.equal(got, ofp8.encode(x))


def test_encode_boundaries_and_odd_lengths():
    x = ofp8.boundary_f32()
    for n in (x.numel(), x.numel() - 1, 3, 1):
        got = fp8_encode(x[:n].to(DEV)).cpu()
        assert torch.equal(got, ofp8.encode(x[:n])), n


def test_decode_all_codes():
    c = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    got = fp8_decode(c.to(DEV)).cpu()
    want = ofp8.decode(c)
    assert torch.equal(torch.isnan(got), torch.isnan(want))
    assert torch.equal(torch.nan_to_num(got), torch.nan_to_num(want))


def test_pack_matches_golden_fixture():
    g = np.load(GOLD)
    k = torch.from_numpy(g["k_bits"]).view(torch.bfloat16)
    v = torch.from_numpy(g["v_bits"]).view(torch.bfloat16)
    page, P = int(g["page_tokens"]), int(g["pool_pages"])
    pool = Fp8PagePool(P, k.shape[1], 128, page, DEV)
    table = pool.page_table(g["table"].tolist())
    pool.pack(k.to(DEV), v.to(DEV), table)
    kc, ks, vc, vs = _pool_to_cpu(pool)
    assert np.array_equal(kc.numpy(), g["k_codes"])
    assert np.array_equal(ks.numpy(), g["k_scales"])
    assert np.array_equal(vc.numpy(), g["v_codes"])
    assert np.array_equal(vs.numpy(), g["v_scales"])


@pytest.mark.parametrize("T,H,page,P,seed", [
    (4680, 12, 1560, 6, 0),    # one 1.3B chunk: 3 full pages
    (4680, 40, 1560, 4, 1),    # 14B head count
    (1000, 12, 1560, 2, 2),    # partial single page
    (3121, 5, 1560, 5, 3),     # two pages + 1 token
    (257, 3, 16, 20, 4),       # small pages, many of them
])
def test_pack_unpack_bit_exact(T, H, page, P, seed):
    k = inputs.heavy_tailed_kv(T, H, 128, seed=1000 + seed)
    v = inputs.heavy_tailed_kv(T, H, 128, seed=2000 + seed)
    n_pages = -(-T // page)
    ids = inputs.page_table(n_pages, P, seed=seed)
    pool = Fp8PagePool(P, H, 128, page, DEV)
    table = pool.page_table(ids)
    pool.pack(k.to(DEV), v.to(DEV), table)
    kc, ks, vc, vs = _pool_to_cpu(pool)
    okc, oks = okv.new_pool(P, page, H, 128)
    ovc, ovs = okv.new_pool(P, page, H, 128)
    okv.pack(k, ids, page, okc, oks)
    okv.pack(v, ids, page, ovc, ovs)
    assert torch.equal(kc, okc) and torch.equal(ks, oks)
    assert torch.equal(vc, ovc) and torch.equal(vs, ovs)
    ko, vo = pool.unpack(table, T)
    assert torch.equal(ko.cpu(), okv.unpack(ids, T, page, okc, oks))
    assert torch.equal(vo.cpu(), okv.unpack(ids, T, page, ovc, ovs))


def test_k_only_and_empty():
    k = inputs.heavy_tailed_kv(100, 2, 128, seed=7)
    pool = Fp8PagePool(4, 2, 128, 64, DEV)
    table = pool.page_table([2, 1])
    pool.pack(k.to(DEV), None, table)
    assert int(pool.v_codes.abs().sum()) == 0
    ko = pool.unpack(table, 100, with_v=False)
    okc, oks = okv.new_pool(4, 64, 2, 128)
    okv.pack(k, [2, 1], 64, okc, oks)
    assert torch.equal(ko.cpu(), okv.unpack([2, 1], 100, 64, okc, oks))
    pool.pack(k[:0].to(DEV), None, table)  # n_tokens == 0 is a no-op
    torch.cuda.synchronize()


def test_invalid_device_page_ids_are_skipped():
    """Device-side guard: ids outside the pool are never written."""
    k = inputs.heavy_tailed_kv(48, 2, 128, seed=8)
    pool = Fp8PagePool(3, 2, 128, 16, DEV)
    table = PageTable([0, 1, 2], 3, DEV)
    table.dev = torch.tensor([1, 7, -1], dtype=torch.int32, device=DEV)  # bypass host validation
    pool.pack(k.to(DEV), k.to(DEV), table)
    okc, oks = okv.new_pool(3, 16, 2, 128)
    okv.pack(k, [1, 7, -1], 16, okc, oks)
    assert torch.equal(pool.k_codes.cpu(), okc) and torch.equal(pool.k_scales.cpu(), oks)
    assert int(pool.k_codes[0].abs().sum()) == 0 and int(pool.k_codes[2].abs().sum()) == 0


def test_thirty_layer_workload_properties():
    """Full 30-layer FP8 KV workload: bit-exact on three layers, and the
    round-trip error bound plus 448-at-row-max on every layer."""
    L, T, H, page = 30, 4680, 12, 1560
    ppl = T // page
    P = 2 * L * ppl
    ids = inputs.page_table(L * ppl, P, seed=7)
    pool = Fp8PagePool(P, H, 128, page, DEV)
    check = {0, 15, 29}
    for layer in range(L):
        k, v = inputs.kv_layer(layer)
        t = pool.page_table(ids[layer * ppl:(layer + 1) * ppl])
        pool.pack(k.to(DEV), v.to(DEV), t)
        ko, vo = pool.unpack(t, T)
        for x, xo, codes_pool in ((k, ko, pool.k_codes), (v, vo, pool.v_codes)):
            xd = x.to(DEV).float()
            xo = xo.float()
            assert float((xo - xd).abs().max()) <= float(xd.abs().max()) * 2.0 ** -4 * 1.01
            if layer in check:
                c, s = okv.quantize_rows(x)
                assert torch.equal(xo.cpu().to(torch.bfloat16), okv.dequantize_rows(c, s))


def test_thirty_layer_single_launch_bit_exact():
    """The launch the headline times: one pack of all 30 layers' K and V (140 400 tokens) into 90 pages
    of a 180-page pool at the seeded page table, then one gather-dequant of the same 90 pages.  Codes and
    scales on every one of the 90 pages, and both bf16 outputs, equal the oracle's bit for bit; the other
    90 pages of the pool stay untouched."""
    L, T, H, page = 30, 4680, 12, 1560
    ppl = T // page
    n_pages = L * ppl
    P = 2 * n_pages
    n = L * T
    ids = inputs.page_table(n_pages, P, seed=7)
    print(f"[case] 30 layers, {n} tokens, {n_pages} of {P} pages, one launch each way", flush=True)
    k_all = torch.cat([inputs.kv_layer(layer)[0] for layer in range(L)])
    v_all = torch.cat([inputs.kv_layer(layer)[1] for layer in range(L)])
    pool = Fp8PagePool(P, H, 128, page, DEV)
    table = pool.page_table(ids)
    kd, vd = k_all.to(DEV), v_all.to(DEV)
    pool.pack(kd, vd, table)
    ko, vo = pool.unpack(table, n)
    del kd, vd
    unused = sorted(set(range(P)) - set(ids))
    for x, xo, codes_pool, scales_pool in ((k_all, ko, pool.k_codes, pool.k_scales),
                                          (v_all, vo, pool.v_codes, pool.v_scales)):
        c, s = okv.quantize_rows(x)
        assert torch.equal(codes_pool[ids].cpu(), c.view(n_pages, page, H, 128))
        assert torch.equal(scales_pool[ids].cpu(), s.view(n_pages, page, H).transpose(1, 2))
        assert int(codes_pool[unused].abs().sum()) == 0 and int(scales_pool[unused].abs().sum()) == 0
        assert torch.equal(xo.cpu(), okv.dequantize_rows(c, s))
        del c, s


@pytest.mark.parametrize("T,H,heavy", [(4680, 12, True), (4680, 40, False), (37, 3, True), (1, 1, False)])
def test_pertensor_kv_bit_exact(T, H, heavy):
    """The reference's per-tensor FP8 KV mode (common.py:143-164) on [2, T, H, 128]: codes, the fp32 scale
    and the fp32 dequantization equal the oracle bit for bit; all_gather_fp8 on one GPU returns the same."""
    from waveforcing_amd.kv import all_gather_fp8, pack_pertensor, unpack_pertensor

    if heavy:
        kv = torch.stack([inputs.heavy_tailed_kv(T, H, 128, seed=60), inputs.heavy_tailed_kv(T, H, 128, seed=61)])
    else:
        kv = torch.randn((2, T, H, 128), generator=torch.Generator().manual_seed(62)).to(torch.bfloat16)
    print(f"[case] per-tensor KV [2, {T}, {H}, 128] heavy={heavy}", flush=True)
    codes, scale = pack_pertensor(kv.to(DEV))
    deq = unpack_pertensor(codes, scale)
    oc, osc = okv.quantize_tensor(kv)
    assert torch.equal(codes.cpu(), oc) and torch.equal(scale.cpu(), osc)
    assert deq.dtype == torch.float32 and torch.equal(deq.cpu(), okv.dequantize_tensor(oc, osc))
    gathered = all_gather_fp8(kv.to(DEV))
    assert len(gathered) == 1 and torch.equal(gathered[0], deq)


def test_pertensor_kv_zero_tensor_takes_the_scale_floor():
    from waveforcing_amd.kv import pack_pertensor, unpack_pertensor

    kv = torch.zeros((2, 64, 2, 128), dtype=torch.bfloat16, device=DEV)
    codes, scale = pack_pertensor(kv)
    oc, osc = okv.quantize_tensor(kv.cpu())
    assert torch.equal(scale.cpu(), osc) and int(codes.abs().sum()) == 0
    assert int(unpack_pertensor(codes, scale).abs().sum()) == 0
