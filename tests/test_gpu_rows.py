"""GPU parity of the block's row kernels (norms, modulation, residuals, per-token quant).

The kernels run on a row engine whose shape (lanes per row, chunks per lane)
is picked from the row width, so the widths below cover every shape: 64 and
1024 (one wave, 1 and 2 chunks per lane), 1536 (3), 1544 and 2048 (4, the
first ragged), 2056 (a workgroup per row, 2), 5120 (3), 8192 (4), 13824 (7)
and 16384 (8).

Bars, against the CPU oracle's torch ops:
* the residual x + bf16(y * gate) (bf16 tensor arithmetic) is bit-exact;
* LayerNorm / RMSNorm outputs differ from torch only by the order of the
  fp32 statistics' sums, i.e. by a flipped bf16 rounding: every difference is
  within 1.5 ulps of the magnitude that rounding acted on (the norm output
  before the shift, or a RoPE pair's norm), and under 1 % of the elements
  differ;
* int8 codes and scales are bit-exact against the oracle's quantization of
  the kernel's own bf16 output.
"""

import pytest
import torch

from oracle import block as ob
from oracle import linear as olin
from waveforcing_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
EPS = 1e-6
WIDTHS = [64, 1024, 1536, 1544, 2048, 2056, 5120, 8192, 13824, 16384]


def _assert_close_bf16(out, ref, mag=None):
    """Every |out - ref| within 1.5 bf16 ulps of ``mag`` (default |ref|): one rounding flip
    of a norm output, carried through the later bf16 steps; and under 1 % of elements differ."""
    out, ref = out.float(), ref.float()
    mag = ref.abs() if mag is None else mag.float().abs()
    d = (out - ref).abs()
    bound = 1.5 * 2.0 ** -7 * torch.maximum(mag, ref.abs())
    frac = (d > 0).float().mean().item()
    worst = (d - bound).max().item()
    assert worst <= 0.0, f"difference exceeds the bound by {worst:.3e}"
    assert frac < 0.01, f"{frac:.4f} of elements differ"


def _mod_rows(F, dim, g):
    """[F, 6, dim] bf16 modulation; chunks i are strided frame rows."""
    return (torch.randn((F, 6, dim), generator=g) * 0.1).to(torch.bfloat16)


@pytest.mark.parametrize("dim", WIDTHS)
def test_ln_modulate_quant(dim):
    g = torch.Generator().manual_seed(dim)
    F, ft = 3, 24
    T = F * ft
    x = (torch.randn((T, dim), generator=g) * 2 + 0.5).to(torch.bfloat16)
    es = _mod_rows(F, dim, g)
    xd, esd = x.to(DEV), es.to(DEV)
    out = torch.empty((T, dim), dtype=torch.bfloat16, device=DEV)
    q = torch.empty((T, dim), dtype=torch.int8, device=DEV)
    qs = torch.empty((T,), dtype=torch.float32, device=DEV)
    shift, scale = esd[:, 0], esd[:, 1]
    _lib.call("wf_ln_modulate_quant", xd.data_ptr(), T, dim, dim, EPS, None, None, shift.data_ptr(),
              scale.data_ptr(), shift.stride(0), ft, out.data_ptr(), dim, q.data_ptr(), qs.data_ptr(),
              _lib.stream_handle(DEV))
    torch.cuda.synchronize()
    fr = torch.arange(T) // ft
    pre = ob.layer_norm(x) * (1 + es[fr, 1])
    ref = pre + es[fr, 0]
    _assert_close_bf16(out.cpu(), ref, pre.float().abs() + es[fr, 0].float().abs())
    oq, os_ = olin.i8_quant_rows(out.cpu())
    assert torch.equal(qs.cpu(), os_)
    assert torch.equal(q.cpu(), oq)


@pytest.mark.parametrize("dim", [1536, 2056, 5120])
@pytest.mark.parametrize("gated", [True, False])
def test_residual_ln_quant(dim, gated):
    """Gated (or plain) residual fused in front of an affine LayerNorm (norm3) or a modulated one."""
    g = torch.Generator().manual_seed(dim + gated)
    F, ft = 3, 16
    T = F * ft
    x = torch.randn((T, dim), generator=g).to(torch.bfloat16)
    y = torch.randn((T, dim), generator=g).to(torch.bfloat16)
    es = _mod_rows(F, dim, g)
    w = (1 + 0.05 * torch.randn((dim,), generator=g)).to(torch.bfloat16)
    b = (0.01 * torch.randn((dim,), generator=g)).to(torch.bfloat16)
    xd, yd, esd, wd, bd = (t.to(DEV) for t in (x, y, es, w, b))
    q = torch.empty((T, dim), dtype=torch.int8, device=DEV)
    qs = torch.empty((T,), dtype=torch.float32, device=DEV)
    out = torch.empty((T, dim), dtype=torch.bfloat16, device=DEV)
    gate = esd[:, 2] if gated else None
    shift, scale = (None, None) if gated else (esd[:, 3], esd[:, 4])
    ld = esd.stride(0)
    _lib.call("wf_gate_residual_ln_quant", xd.data_ptr(), T, dim, dim, yd.data_ptr(), dim, _lib.ptr(gate), ld, EPS,
              _lib.ptr(wd) if gated else None, _lib.ptr(bd) if gated else None, _lib.ptr(shift), _lib.ptr(scale), ld,
              ft, out.data_ptr(), dim, q.data_ptr(), qs.data_ptr(), _lib.stream_handle(DEV))
    torch.cuda.synchronize()
    fr = torch.arange(T) // ft
    xr = x + y * es[fr, 2] if gated else x + y
    assert torch.equal(xd.cpu(), xr), "residual is not bit-exact"
    if gated:
        ref = ob.layer_norm(xr, w, b)
        mag = None
    else:
        pre = ob.layer_norm(xr) * (1 + es[fr, 4])
        ref = pre + es[fr, 3]
        mag = pre.float().abs() + es[fr, 3].float().abs()
    _assert_close_bf16(out.cpu(), ref, mag)
    oq, os_ = olin.i8_quant_rows(out.cpu())
    assert torch.equal(qs.cpu(), os_) and torch.equal(q.cpu(), oq)


@pytest.mark.parametrize("dim", [256, 1536, 2048, 5120, 8192])
@pytest.mark.parametrize("rope", [True, False])
def test_rmsnorm_rope(dim, rope):
    g = torch.Generator().manual_seed(dim + 7 * rope)
    T, hd = 96, 128
    H = dim // hd
    # a strided column view, as q/k inside the fused QKV output
    qkv = torch.randn((T, 3 * dim), generator=g).to(torch.bfloat16)
    w = (1 + 0.05 * torch.randn((dim,), generator=g)).to(torch.bfloat16)
    ang = torch.rand((T, hd // 2), generator=g, dtype=torch.float64) * 6.0
    qkvd, wd = qkv.to(DEV), w.to(DEV)
    cos = torch.cos(ang).float().to(DEV) if rope else None
    sin = torch.sin(ang).float().to(DEV) if rope else None
    xk = qkvd[:, dim:2 * dim]
    _lib.call("wf_rmsnorm_rope", xk.data_ptr(), T, dim, xk.stride(0), hd, EPS, wd.data_ptr(), _lib.ptr(cos),
              _lib.ptr(sin), xk.data_ptr(), xk.stride(0), _lib.stream_handle(DEV))
    torch.cuda.synchronize()
    ref = ob.rms_norm(qkv[:, dim:2 * dim], w)
    mag = None
    if rope:
        # fp32 tables, rotation in fp32 on the bf16 RMSNorm output
        c, s = torch.cos(ang).float(), torch.sin(ang).float()
        r = ref.float().view(T, H, hd // 2, 2)
        a0, a1 = r[..., 0], r[..., 1]
        cc, ss = c.view(T, 1, -1), s.view(T, 1, -1)
        ref = torch.stack([a0 * cc - a1 * ss, a0 * ss + a1 * cc], -1).view(T, dim).to(torch.bfloat16)
        # a rotation moves a one-ulp input difference anywhere within the pair's norm
        mag = torch.sqrt(a0 * a0 + a1 * a1).repeat_interleave(2, -1).view(T, dim)
    out = qkvd.cpu()
    _assert_close_bf16(out[:, dim:2 * dim], ref, mag)
    assert torch.equal(out[:, :dim], qkv[:, :dim]) and torch.equal(out[:, 2 * dim:], qkv[:, 2 * dim:])


@pytest.mark.parametrize("M,K", [(64, 2064), (33, 13824), (17, 16384), (3, 16512)])
def test_act_quant_widths(M, K):
    """Per-token int8 quant at the widths of each row-engine shape and past it (the two-read kernel)."""
    g = torch.Generator().manual_seed(K)
    x = (torch.randn((M, K), generator=g) * 3).to(torch.bfloat16)
    x[:, K // 3] *= 40
    q = torch.empty((M, K), dtype=torch.int8, device=DEV)
    s = torch.empty((M,), dtype=torch.float32, device=DEV)
    xd = x.to(DEV)
    _lib.call("wf_act_quant_i8", xd.data_ptr(), M, K, K, q.data_ptr(), s.data_ptr(), _lib.stream_handle(DEV))
    torch.cuda.synchronize()
    oq, os_ = olin.i8_quant_rows(x)
    assert torch.equal(s.cpu(), os_) and torch.equal(q.cpu(), oq)


def test_gate_residual_strided_gate():
    g = torch.Generator().manual_seed(3)
    F, ft, dim = 3, 10, 1536
    T = F * ft
    x = torch.randn((T, dim), generator=g).to(torch.bfloat16)
    y = torch.randn((T, dim), generator=g).to(torch.bfloat16)
    es = _mod_rows(F, dim, g)
    xd, yd, esd = x.to(DEV), y.to(DEV), es.to(DEV)
    gate = esd[:, 5]
    _lib.call("wf_gate_residual", xd.data_ptr(), dim, yd.data_ptr(), dim, gate.data_ptr(), gate.stride(0), T, dim, ft,
              _lib.stream_handle(DEV))
    torch.cuda.synchronize()
    fr = torch.arange(T) // ft
    assert torch.equal(xd.cpu(), x + y * es[fr, 5])


@pytest.mark.parametrize("dim", [64, 1536, 2056, 5120, 13824])
@pytest.mark.parametrize("form", ["gated_mod", "mod", "plain_res_mod", "gated_affine"])
def test_ln_forms_match_the_general_kernel(dim, form):
    """The LayerNorm launches of the block (int8 output only) run kernels specialized at compile time;
    the same call with a bf16 output as well runs the run-time form.  Codes, scales and the in-place
    residual must agree bit for bit."""
    g = torch.Generator().manual_seed(7 * dim + len(form))
    F, ft = 3, 20
    T = F * ft
    x = torch.randn((T, dim), generator=g).to(torch.bfloat16).to(DEV)
    y = torch.randn((T, dim), generator=g).to(torch.bfloat16).to(DEV)
    es = _mod_rows(F, dim, g).to(DEV)
    w = (1 + 0.05 * torch.randn((dim,), generator=g)).to(torch.bfloat16).to(DEV)
    b = (0.01 * torch.randn((dim,), generator=g)).to(torch.bfloat16).to(DEV)
    res_y = None if form == "mod" else y
    gate = es[:, 2] if form.startswith("gated") else None
    aff = form == "gated_affine"
    shift, scale = (None, None) if aff else (es[:, 0], es[:, 1])
    ld = es.stride(0)
    got = []
    for with_out in (False, True):
        xd = x.clone()
        q = torch.empty((T, dim), dtype=torch.int8, device=DEV)
        qs = torch.empty((T,), dtype=torch.float32, device=DEV)
        out = torch.empty((T, dim), dtype=torch.bfloat16, device=DEV) if with_out else None
        _lib.call("wf_gate_residual_ln_quant", xd.data_ptr(), T, dim, dim, _lib.ptr(res_y), dim, _lib.ptr(gate), ld,
                  EPS, _lib.ptr(w) if aff else None, _lib.ptr(b) if aff else None, _lib.ptr(shift), _lib.ptr(scale),
                  ld, ft, _lib.ptr(out), dim if with_out else 0, q.data_ptr(), qs.data_ptr(), _lib.stream_handle(DEV))
        got.append((xd, q, qs))
    torch.cuda.synchronize()
    (x0, q0, s0), (x1, q1, s1) = got
    assert torch.equal(x0, x1) and torch.equal(q0, q1) and torch.equal(s0, s1)
