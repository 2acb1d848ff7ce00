"""scaled_dot_product_attention and causal-mask ops on the `applegpu` torch
device (the remaining CPU fallbacks around the hot path: the reference
registers none of them, backend_cpp/applegpu_backend.cpp:432-435, 753-764).

SDPA without a mask or dropout is routed by _fused_sdp_choice to the
overrideable backend: the fused attention kernel forward, a device-GEMM
backward that recomputes the probabilities.  Values against torch CPU: fp32
within the 1e-3 attention bar, fp16/bf16 within 1e-2; masks bit-exact."""
import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev(gpu):
    import torch
    from applegpu_runtime.cpp_backend import load_cpp_backend
    load_cpp_backend()
    return torch


def _fallbacks():
    from applegpu_runtime.cpp_backend import fallback_count
    return fallback_count()


@pytest.mark.parametrize("B,H,Tq,Tk,D,causal,scale", [
    (2, 4, 128, 128, 64, True, None),
    (2, 4, 128, 128, 64, False, None),
    (1, 12, 100, 100, 64, True, 0.3),
    (2, 2, 16, 48, 32, False, None),
    (2, 2, 16, 48, 128, True, None),   # top-left causal with Tq < Tk
    (3, 50, 64, 64, None, True, None),  # 3-D [B*H, T, D] operands
])
def test_sdpa_forward_and_backward_match_cpu(torch_dev, B, H, Tq, Tk, D, causal, scale):
    torch = torch_dev
    F = torch.nn.functional
    torch.manual_seed(5)
    if D is None:
        shp_q, shp_k = (B, Tq, H), (B, Tk, H)
    else:
        shp_q, shp_k = (B, H, Tq, D), (B, H, Tk, D)
    q, k, v = torch.randn(shp_q), torch.randn(shp_k), torch.randn(shp_k)
    go = torch.randn(shp_q)
    qc, kc, vc = (t.clone().requires_grad_(True) for t in (q, k, v))
    ref = F.scaled_dot_product_attention(qc, kc, vc, is_causal=causal, scale=scale)
    ref.backward(go)
    qd, kd, vd = (t.to("applegpu").requires_grad_(True) for t in (q, k, v))
    assert torch._fused_sdp_choice(qd, kd, vd, is_causal=causal) == 4   # overrideable
    before = _fallbacks()
    out = F.scaled_dot_product_attention(qd, kd, vd, is_causal=causal, scale=scale)
    out.backward(go.to("applegpu"))
    assert _fallbacks() == before
    assert rel_err(out.detach().cpu().numpy(), ref.detach().numpy()) < 1e-3
    for a, b in ((qd, qc), (kd, kc), (vd, vc)):
        assert rel_err(a.grad.cpu().numpy(), b.grad.numpy()) < 1e-3


@pytest.mark.parametrize("dt", ["float16", "bfloat16"])
def test_sdpa_16bit_inference(torch_dev, dt):
    torch = torch_dev
    F = torch.nn.functional
    torch.manual_seed(6)
    q, k, v = (torch.randn(2, 12, 128, 64).to(getattr(torch, dt)) for _ in range(3))
    ref = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), is_causal=True)
    with torch.no_grad():
        got = F.scaled_dot_product_attention(q.to("applegpu"), k.to("applegpu"), v.to("applegpu"), is_causal=True)
    assert got.dtype == getattr(torch, dt)
    assert rel_err(got.float().cpu().numpy(), ref.numpy()) < 1e-2


def test_sdpa_with_mask_takes_the_math_path(torch_dev):
    torch = torch_dev
    F = torch.nn.functional
    torch.manual_seed(7)
    q, k, v = (torch.randn(1, 2, 8, 16) for _ in range(3))
    mask = torch.rand(8, 8) > 0.3
    mask[:, 0] = True
    ref = F.scaled_dot_product_attention(q, k, v, attn_mask=mask)
    qd, kd, vd = (t.to("applegpu") for t in (q, k, v))
    assert torch._fused_sdp_choice(qd, kd, vd, attn_mask=mask.to("applegpu")) == 0   # math
    got = F.scaled_dot_product_attention(qd, kd, vd, attn_mask=mask.to("applegpu"))
    assert rel_err(got.cpu().numpy(), ref.numpy()) < 1e-3


def test_causal_mask_ops_run_on_device(torch_dev):
    """The GPT-2 recipe's explicit mask: triu/tril, masked_fill(-inf), where."""
    torch = torch_dev
    torch.manual_seed(8)
    s = torch.randn(2, 3, 16, 16)
    mask = torch.triu(torch.ones(16, 16), diagonal=1).bool()
    sd = s.to("applegpu")
    before = _fallbacks()
    md = torch.triu(torch.ones(16, 16).to("applegpu"), diagonal=1).bool()
    a = sd.masked_fill(md, float("-inf"))
    b = torch.where(md, torch.zeros(16, 16).to("applegpu"), sd)
    c = torch.tril(sd, diagonal=-2)
    d = sd.clone()
    d.masked_fill_(md, 0.0)
    assert _fallbacks() == before
    np.testing.assert_array_equal(a.cpu().numpy(), s.masked_fill(mask, float("-inf")).numpy())
    np.testing.assert_array_equal(b.cpu().numpy(), torch.where(mask, torch.zeros(16, 16), s).numpy())
    np.testing.assert_array_equal(c.cpu().numpy(), torch.tril(s, diagonal=-2).numpy())
    np.testing.assert_array_equal(d.cpu().numpy(), s.masked_fill(mask, 0.0).numpy())
    np.testing.assert_array_equal(md.cpu().numpy(), mask.numpy())
