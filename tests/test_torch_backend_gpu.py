"""The PyTorch PrivateUse1 device `applegpu` (applegpu_runtime.cpp_backend),
checked against PyTorch CPU eager as the reference's own PrivateUse1 tests do
(python/tests/test_cpp_backend.py:92-216, 267-371)."""
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


def test_tensor_round_trip_and_views(torch_dev):
    torch = torch_dev
    a = torch.arange(24, dtype=torch.float32).reshape(4, 6)
    d = a.to("applegpu")
    assert d.device.type == "applegpu"
    np.testing.assert_array_equal(d.cpu().numpy(), a.numpy())
    np.testing.assert_array_equal(d.t().cpu().numpy(), a.t().numpy())
    np.testing.assert_array_equal(d[1:3, 2:5].cpu().numpy(), a[1:3, 2:5].numpy())
    np.testing.assert_array_equal((d[1:3, 2:5] * 2).cpu().numpy(), (a[1:3, 2:5] * 2).numpy())
    z = torch.zeros(3, 5, device="applegpu")
    z.fill_(1.5)
    np.testing.assert_array_equal(z.cpu().numpy(), np.full((3, 5), 1.5, np.float32))


def test_linear_forward_matches_cpu(torch_dev):
    # python/tests/test_cpp_backend.py:121-133 (1e-5)
    torch = torch_dev
    torch.manual_seed(42)
    lin = torch.nn.Linear(4, 3)
    x = torch.randn(2, 4)
    want = lin(x)
    got = lin.to("applegpu")(x.to("applegpu")).cpu()
    assert rel_err(got.detach().numpy(), want.detach().numpy()) < 1e-5


@pytest.mark.parametrize("op", ["layer_norm", "gelu", "gelu_tanh", "softmax", "log_softmax", "relu"])
def test_ops_match_cpu(torch_dev, op):
    torch = torch_dev
    import torch.nn.functional as F
    torch.manual_seed(1)
    x = torch.randn(8, 768)
    fns = {
        "layer_norm": lambda t: F.layer_norm(t, (768,), torch.ones(768, device=t.device) * 1.5,
                                             torch.full((768,), 0.25, device=t.device)),
        "gelu": lambda t: F.gelu(t), "gelu_tanh": lambda t: F.gelu(t, approximate="tanh"),
        "softmax": lambda t: F.softmax(t, -1), "log_softmax": lambda t: F.log_softmax(t, -1),
        "relu": lambda t: F.relu(t),
    }
    want = fns[op](x).numpy()
    got = fns[op](x.to("applegpu")).cpu().numpy()
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_mlp_config1_training_matches_cpu_without_fallback(torch_dev):
    """Config 1: Linear(64,128)-ReLU-Linear(128,10), MSE, SGD(lr=0.01), 3 steps,
    loss and parameters vs CPU; no op may take the CPU fallback."""
    torch = torch_dev
    from applegpu_runtime.cpp_backend import fallback_count

    def make():
        torch.manual_seed(42)
        return torch.nn.Sequential(torch.nn.Linear(64, 128), torch.nn.ReLU(), torch.nn.Linear(128, 10))

    torch.manual_seed(42)
    x, y = torch.randn(32, 64), torch.randn(32, 10)
    cpu, dev = make(), make().to("applegpu")
    xd, yd = x.to("applegpu"), y.to("applegpu")
    oc = torch.optim.SGD(cpu.parameters(), lr=0.01)
    od = torch.optim.SGD(dev.parameters(), lr=0.01)
    before = fallback_count()
    for step in range(3):
        oc.zero_grad()
        lc = torch.nn.functional.mse_loss(cpu(x), y)
        lc.backward()
        oc.step()
        od.zero_grad()
        ld = torch.nn.functional.mse_loss(dev(xd), yd)
        ld.backward()
        od.step()
        assert abs(ld.item() - lc.item()) <= 1e-4 * abs(lc.item()), step
    assert fallback_count() == before, "an op of the MLP training step ran on the CPU"
    for pc, pd in zip(cpu.parameters(), dev.parameters()):
        assert rel_err(pd.detach().cpu().numpy(), pc.detach().numpy()) < 1e-5


def test_transformer_block_matches_cpu(torch_dev):
    """python/tests/test_cpp_backend.py:267-308: a pre-LN attention block (1e-3)."""
    torch = torch_dev
    import torch.nn.functional as F
    torch.manual_seed(5)
    T, d, H = 16, 64, 4
    x = torch.randn(T, d)
    w_qkv, b_qkv = torch.randn(d, 3 * d) * 0.1, torch.zeros(3 * d)
    w_o = torch.randn(d, d) * 0.1
    g, b = torch.ones(d), torch.zeros(d)

    def block(t, dev):
        m = lambda a: a.to(dev)  # noqa: E731
        h = F.layer_norm(t, (d,), m(g), m(b))
        qkv = h @ m(w_qkv) + m(b_qkv)
        q, k, v = (qkv[:, i * d:(i + 1) * d].reshape(T, H, d // H).transpose(0, 1) for i in range(3))
        s = torch.matmul(q, k.transpose(1, 2).contiguous()) * (1.0 / (d // H) ** 0.5)
        a = torch.matmul(F.softmax(s, -1), v)
        return t + a.transpose(0, 1).reshape(T, d) @ m(w_o)

    want = block(x, "cpu")
    got = block(x.to("applegpu"), "applegpu").cpu()
    assert rel_err(got.numpy(), want.numpy()) < 1e-3
