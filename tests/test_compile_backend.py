"""torch.compile backend: the op-list serializer, the op-list semantics (the
numpy restatement in oracle/compiled_graph.py) and the device executor
(applegpu_eager_execute_graph), after python/tests/test_compile_backend.py
of the reference.

CPU tests: hand-assembled op lists decode to known records; aot_autograd's
forward and backward graphs of the reference's test models serialize, and
the decoded op lists run on numpy reproduce what torch CPU computes for
the same graphs; the C ABI rejects malformed op lists before touching a
device.  GPU tests: the device executor against the numpy op-list runner
on the same inputs, and torch.compile on the `applegpu` device against
torch CPU (the reference's cases: mm, add, relu, addmm, Linear, backward,
MLP forward, an MLP SGD step).
"""
import ctypes
import os
import struct
import subprocess
import sys

import numpy as np
import pytest
import torch

from conftest import rel_err
from oracle import compiled_graph as CG

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "applegpu-runtime_amd")
LIB = os.path.join(PKG, "applegpu_runtime", "libapplegpu_core.so")
RNG = np.random.default_rng(7373)


def _backend():
    sys.path.insert(0, PKG) if PKG not in sys.path else None
    from applegpu_runtime import compile_backend as CB
    return CB


def _enc(code, ins, dims=(), params=(), dtype=0):
    return _backend()._encode(code, list(ins), list(dims), dtype, list(params))


# ── CPU: format and serializer ──────────────────────────────────────────────
def test_decode_known_bytes():
    """Byte layout of compiled_graph.rs:7-9, assembled by hand."""
    raw = bytes([13, 3, 2, 0, 0, 0, 1, 0, 2]) + struct.pack("<QQ", 4, 3) + bytes([0, 0])
    raw += bytes([7, 2, 3, 0, 1, 0, 1]) + struct.pack("<Q", 5) + bytes([0, 1]) + struct.pack("<f", 0.5)
    ops = CG.decode(raw)
    assert ops == [
        {"code": 13, "inputs": [2, 0, 1], "dims": [4, 3], "dtype": 0, "params": []},
        {"code": 7, "inputs": [3, 1], "dims": [5], "dtype": 0, "params": [0.5]},
    ]
    assert _enc(13, [2, 0, 1], [4, 3]) + _enc(7, [3, 1], [5], [0.5]) == raw
    with pytest.raises(ValueError):
        CG.decode(raw[:-1])


def _capture(fn, *inputs):
    """aot_autograd forward and backward graphs of fn on CPU tensors, each
    with the inputs it was called with (a capturing compiler that runs the
    graph module itself)."""
    from torch._functorch.aot_autograd import aot_function, make_boxed_func
    seen = []

    def compiler(gm, example_inputs):
        def run(args):
            seen.append((gm, [a.detach().clone() if isinstance(a, torch.Tensor) else a for a in args]))
            return gm(*args)
        run._boxed_call = True
        return run

    f = aot_function(fn, fw_compiler=compiler, bw_compiler=compiler)
    out = f(*inputs)
    return out, seen


def _check_graph(gm, args):
    CB = _backend()
    ser = CB.serialize_graph(gm)
    assert ser is not None, gm.graph
    ops, n_ph, outs = ser
    assert n_ph == len(args)
    want = gm(*args)
    want = list(want) if isinstance(want, (tuple, list)) else [want]
    real = [i for i in outs if i != CB.NONE_OUTPUT]
    got = CG.run(ops, [a.numpy() if isinstance(a, torch.Tensor) else None for a in args], real)
    want = [w for w, o in zip(want, outs) if o != CB.NONE_OUTPUT]
    assert len(got) == len(want)
    for g, w in zip(got, want):
        w = w.detach().numpy()
        assert g.size == w.size
        assert rel_err(np.reshape(g, w.shape), w) < 1e-5
    return CG.decode(ops)


def test_mlp_graphs_serialize_and_match_torch():
    torch.manual_seed(0)
    fc1, fc2 = torch.nn.Linear(8, 16), torch.nn.Linear(16, 4)
    x = torch.randn(2, 8)
    params = [p.detach().clone().requires_grad_(True) for p in (fc1.weight, fc1.bias, fc2.weight, fc2.bias)]

    def mlp(x, w1, b1, w2, b2):
        h = torch.relu(torch.nn.functional.linear(x, w1, b1))
        return torch.nn.functional.linear(h, w2, b2)

    out, seen = _capture(mlp, x, *params)
    out.sum().backward()
    assert len(seen) == 2  # forward, backward
    codes = set()
    for gm, args in seen:
        codes |= {op["code"] for op in _check_graph(gm, args)}
    assert {CG.ADDMM, CG.RELU, CG.TRANSPOSE, CG.MATMUL, CG.SUM_DIM, CG.THRESHOLD_BACKWARD} <= codes


def test_elementwise_graph_with_scalars_and_views():
    def f(a, b):
        c = (a * 2.5 - b) / (b * b)
        return (-c).relu().reshape(-1, 4).sum(0, keepdim=True), (a @ b.t()).mean()

    a, b = torch.randn(6, 4), torch.rand(6, 4) + 0.5

    from torch._functorch.aot_autograd import aot_function
    seen = []

    def compiler(gm, example_inputs):
        seen.append(gm)
        return gm

    aot_function(f, fw_compiler=compiler)(a, b)
    (gm,) = seen
    ops = _check_graph(gm, [a, b])
    assert {CG.SCALAR_MUL, CG.SUB, CG.DIV, CG.NEG, CG.VIEW, CG.MEAN_ALL} <= {o["code"] for o in ops}


def test_unexpressible_graph_is_not_serialized():
    """Ops without a code, alpha != 1, a scalar addend and sums over several
    dims make the graph run as a module instead of computing something else."""
    from torch._functorch.aot_autograd import aot_function
    CB = _backend()
    for fn in (lambda a: torch.exp(a), lambda a: torch.add(a, a, alpha=2.0), lambda a: a + 1.5,
               lambda a: a.sum((0, 1))):
        seen = []
        aot_function(fn, fw_compiler=lambda gm, ex: seen.append(gm) or gm)(torch.randn(3, 4))
        assert CB.serialize_graph(seen[0]) is None


def _abi(code):
    out = subprocess.run([sys.executable, "-c", code, LIB], capture_output=True, text=True, timeout=120)
    return out.stdout.strip()


def test_abi_rejects_malformed_op_lists_without_a_device():
    """Parsing comes first: truncated lists, forward references, unknown op
    codes and out-of-range outputs fail with a message; a well-formed list
    then fails only for want of a device."""
    prelude = ("import ctypes,sys; lib=ctypes.CDLL(sys.argv[1]);"
               "lib.applegpu_eager_last_error.restype=ctypes.c_char_p;"
               "ids=(ctypes.c_uint64*2)(1,2); oi=(ctypes.c_uint16*1)(2); ot=(ctypes.c_uint64*1)();"
               "op=(ctypes.c_void_p*1)();")

    def call(raw, outs=2):
        return _abi(prelude + f"raw={raw!r}; oi[0]={outs};"
                    "r=lib.applegpu_eager_execute_graph(raw,len(raw),ids,2,oi,1,ot,op);"
                    "print(r, lib.applegpu_eager_last_error().decode())")

    good = _enc(0, [0, 1], [3])
    assert call(good[:-1]).startswith("-1 compiled graph failed: op list truncated")
    assert "reads node 5" in call(_enc(0, [0, 5], [3]))
    assert "unsupported op: 99" in call(_enc(99, [0], [3]))
    assert "output 3 out of range" in call(good, outs=3)
    assert "needs 2" in call(_enc(0, [0], [3]))
    r = call(good)
    assert r.startswith("-1") and "device" in r


# ── GPU: the device executor ────────────────────────────────────────────────
def _f32(*shape):
    return RNG.standard_normal(shape).astype(np.float32)


@pytest.mark.gpu
def test_executor_matches_numpy_runner(gpu):
    """One op list touching every op code, with outputs that are inputs,
    views, the same node twice and a fused addmm + relu chain."""
    from applegpu_runtime import eager as E
    from applegpu_runtime._native import lib
    x, w, b, g = _f32(32, 48), _f32(48, 24), _f32(24), _f32(32, 24)
    ins = [x, w, b, g]
    raw = b"".join([
        _enc(CG.ADDMM, [2, 0, 1], [32, 24]),             # 4  x @ w + b
        _enc(CG.RELU, [4], [32, 24]),                    # 5
        _enc(CG.THRESHOLD_BACKWARD, [3, 5], [32, 24], [0.0]),  # 6
        _enc(CG.TRANSPOSE, [0], [48, 32]),               # 7  x^T (view)
        _enc(CG.MATMUL, [7, 6], [48, 24]),               # 8  x^T @ g'
        _enc(CG.SUM_DIM, [6], [1, 24], [0.0, 1.0]),      # 9
        _enc(CG.SUM_DIM, [6], [32], [-1.0, 0.0]),        # 10
        _enc(CG.SCALAR_MUL, [8], [48, 24], [-0.25]),     # 11
        _enc(CG.ADD, [1, 11], [48, 24]),                 # 12 w + (-0.25) x^T g'
        _enc(CG.SUB, [5, 3], [32, 24]),                  # 13
        _enc(CG.MUL, [13, 13], [32, 24]),                # 14
        _enc(CG.MEAN_ALL, [14], [1]),                    # 15
        _enc(CG.DIV, [3, 2], [32, 24]),                  # 16 g / b
        _enc(CG.NEG, [16], [32, 24]),                    # 17
        _enc(CG.VIEW, [17], [24, 32]),                   # 18
        _enc(CG.VIEW, [7], [32, 48]),                    # 19 reshape of a transposed view
        _enc(CG.IDENTITY, [2], [24]),                    # 20 an input passed through
        _enc(CG.TRANSPOSE, [2], [24]),                   # 21 t of a 1-D node
    ])
    outs = [5, 6, 8, 9, 10, 12, 15, 18, 19, 20, 21, 12, 7]
    want = CG.run(raw, ins, outs)
    ts = [E.from_numpy(a) for a in ins]
    in_ids = (ctypes.c_uint64 * 4)(*[t.id for t in ts])
    oi = (ctypes.c_uint16 * len(outs))(*outs)
    ot = (ctypes.c_uint64 * len(outs))()
    op = (ctypes.c_void_p * len(outs))()
    n = lib.applegpu_eager_execute_graph(raw, len(raw), in_ids, 4, oi, len(outs), ot, op)
    assert n == len(outs), lib.applegpu_eager_last_error()
    assert ot[9] == ts[2].id and ot[10] == ts[2].id   # inputs come back as their own ids
    assert ot[5] == ot[11]                            # one node, one id
    got = []
    for i in range(len(outs)):
        t = E.EagerTensor(int(ot[i]), None)
        got.append(t.numpy())
        t.id = 0                                      # read only; freed below
    for tid in {int(ot[i]) for i in range(len(outs))} - {t.id for t in ts}:
        lib.applegpu_eager_free(tid)
    for i, (gv, wv) in enumerate(zip(got, want)):
        tol = 1e-3 if outs[i] in (8, 12) else 1e-5   # GEMM bar for the matmul outputs
        assert gv.shape == np.shape(wv) or (outs[i] == 15 and gv.size == 1), (i, gv.shape, np.shape(wv))
        assert rel_err(np.reshape(gv, np.shape(wv)), wv) < tol, i


def _sub(code):
    """torch.compile in a fresh process (aot_autograd state is per process,
    as the reference's tests do); prints PASS."""
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([PKG, ROOT, os.environ.get("PYTHONPATH", "")]))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0 and r.stdout.strip().endswith("PASS"), r.stdout[-2000:] + r.stderr[-4000:]


_PRE = """
import torch
from applegpu_runtime.cpp_backend import load_cpp_backend, fallback_count
load_cpp_backend()
from applegpu_runtime import compile_backend as CB
from applegpu_runtime._native import lib
runners = []
_orig = CB.CompiledGraphRunner.__init__
def _init(self, gm):
    _orig(self, gm)
    runners.append(self)
CB.CompiledGraphRunner.__init__ = _init
calls = [0]
_ex = lib.applegpu_eager_execute_graph
"""


@pytest.mark.gpu
def test_compile_single_ops_match_cpu(gpu):
    _sub(_PRE + """
torch.manual_seed(0)
cases = [
    (lambda a, b: torch.mm(a, b), (torch.randn(4, 3), torch.randn(3, 5))),
    (lambda a, b: a + b, (torch.randn(4, 3), torch.randn(4, 3))),
    (lambda a: torch.relu(a), (torch.randn(6, 7),)),
    (lambda bias, x, w: torch.addmm(bias, x, w), (torch.randn(2), torch.randn(4, 3), torch.randn(3, 2))),
]
for fn, args in cases:
    want = fn(*args)
    got = torch.compile(fn, backend=CB.applegpu_compile_backend)(*[a.to('applegpu') for a in args])
    assert got.device.type == 'applegpu'
    assert torch.allclose(got.cpu(), want, atol=1e-4), (fn, got.cpu(), want)
    torch._dynamo.reset()
assert runners and all(r.serialized for r in runners)
print("PASS")
""")


@pytest.mark.gpu
def test_compile_linear_and_mlp_forward(gpu):
    _sub(_PRE + """
torch.manual_seed(42)
layer = torch.nn.Linear(8, 4)
x = torch.randn(2, 8)
want = layer(x)
got = torch.compile(layer.to('applegpu'), backend=CB.applegpu_compile_backend)(x.to('applegpu'))
assert torch.allclose(got.cpu(), want, atol=1e-4)
class MLP(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.fc1 = torch.nn.Linear(64, 256)
        self.fc2 = torch.nn.Linear(256, 10)
    def forward(self, x):
        return self.fc2(torch.relu(self.fc1(x)))
m = MLP()
x = torch.randn(32, 64)
want = m(x)
got = torch.compile(m.to('applegpu'), backend=CB.applegpu_compile_backend)(x.to('applegpu'))
assert torch.allclose(got.cpu(), want, atol=1e-4), (got.cpu() - want).abs().max()
assert all(r.serialized for r in runners)
print("PASS")
""")


@pytest.mark.gpu
def test_compile_backward_and_training_step(gpu):
    """The reference's backward and SGD-step cases, plus several steps of the
    C1 MLP with gradients checked against CPU autograd each step."""
    _sub(_PRE + """
torch.manual_seed(1)
x = torch.randn(4, 3, requires_grad=True)
w = torch.randn(3, 2, requires_grad=True)
torch.mm(x, w).sum().backward()
xd = x.detach().to('applegpu').requires_grad_(True)
wd = w.detach().to('applegpu').requires_grad_(True)
f = torch.compile(lambda a, b: torch.mm(a, b), backend=CB.applegpu_compile_backend)
f(xd, wd).sum().backward()
assert torch.allclose(xd.grad.cpu(), x.grad, atol=1e-4) and torch.allclose(wd.grad.cpu(), w.grad, atol=1e-4)
torch._dynamo.reset()

class MLP(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.fc1 = torch.nn.Linear(64, 128)
        self.fc2 = torch.nn.Linear(128, 10)
    def forward(self, x):
        return self.fc2(torch.relu(self.fc1(x)))
torch.manual_seed(42)
ref = MLP()
dev = MLP()
dev.load_state_dict(ref.state_dict())
dev = dev.to('applegpu')
cm = torch.compile(dev, backend=CB.applegpu_compile_backend)
ro = torch.optim.SGD(ref.parameters(), lr=0.01)
do = torch.optim.SGD(dev.parameters(), lr=0.01)
for step in range(3):
    xs, ys = torch.randn(32, 64), torch.randn(32, 10)
    ro.zero_grad(); do.zero_grad()
    lr_ = torch.nn.functional.mse_loss(ref(xs), ys); lr_.backward(); ro.step()
    ld = torch.nn.functional.mse_loss(cm(xs.to('applegpu')), ys.to('applegpu')); ld.backward(); do.step()
    assert abs(ld.item() - lr_.item()) < 1e-4 * max(1.0, abs(lr_.item())), (step, ld.item(), lr_.item())
    for p, q in zip(dev.parameters(), ref.parameters()):
        assert (p.detach().cpu() - q.detach()).abs().max().item() < 1e-4, step
assert len(runners) >= 2 and all(r.serialized for r in runners), [r.gm.graph for r in runners if not r.serialized]
print("PASS")
""")
