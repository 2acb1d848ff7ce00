"""torch.compile backend for the `applegpu` device: one C-ABI call per graph.

Same entry point and wire format as the reference
(python/applegpu_runtime/compile_backend.py:789-1092): aot_autograd hands
each forward and backward FX graph to a compiler that serializes it into the
op list `applegpu_eager_execute_graph` reads (crates/core/src/
compiled_graph.rs:7-9); every call of the compiled function is then one
FFI call.  On this backend the executor records the whole op list into the
lazy graph and runs it as one fusion-planned launch sequence (addmm + relu
is one GEMM with a fused epilogue) on the library stream, so a call neither
waits for the device nor copies outputs: results come back as `applegpu`
tensors that own the runtime's buffers (torch.ops.applegpu.wrap_eager).

Graphs holding an op the op list cannot express run as plain FX graph
modules on the device instead (the aten kernels of the PrivateUse1 shim);
`CompiledGraphRunner.serialized` says which path a graph took.

Usage:
    from applegpu_runtime.compile_backend import applegpu_compile_backend
    compiled = torch.compile(model, backend=applegpu_compile_backend)
"""
from __future__ import annotations

import ctypes
import struct

import torch

# Op codes of the wire format (crates/core/src/compiled_graph.rs:43-57).
OP_ADD, OP_SUB, OP_MUL, OP_DIV, OP_MATMUL, OP_RELU, OP_NEG, OP_THRESHOLD_BACKWARD, OP_SCALAR_MUL, OP_MEAN_ALL, \
    OP_SUM_DIM, OP_TRANSPOSE, OP_VIEW, OP_ADDMM = range(14)
OP_IDENTITY = 255
NONE_OUTPUT = 0xFFFF  # output slot holding None (a gradient that does not exist)

_WIRE = {torch.float32: 0, torch.float16: 1, torch.float64: 2, torch.int8: 3, torch.int16: 4, torch.int32: 5,
         torch.int64: 6, torch.uint8: 7, torch.bool: 9, torch.bfloat16: 10}

aten = torch.ops.aten
# target -> (op code, number of leading tensor arguments)
_TENSOR_OPS = {
    aten.add.Tensor: (OP_ADD, 2), aten.sub.Tensor: (OP_SUB, 2), aten.mul.Tensor: (OP_MUL, 2),
    aten.div.Tensor: (OP_DIV, 2), aten.mm.default: (OP_MATMUL, 2), aten.relu.default: (OP_RELU, 1),
    aten.neg.default: (OP_NEG, 1), aten.threshold_backward.default: (OP_THRESHOLD_BACKWARD, 2),
    aten.t.default: (OP_TRANSPOSE, 1), aten.addmm.default: (OP_ADDMM, 3), aten.mean.default: (OP_MEAN_ALL, 1),
}
_IDENTITY_OPS = {aten.detach.default, aten.alias.default}
_VIEW_OPS = {aten.view.default, aten.reshape.default, aten._unsafe_view.default}


class _Unsupported(Exception):
    pass


def _meta(node):
    val = node.meta.get("val") if isinstance(node, torch.fx.Node) else None
    return val if isinstance(val, torch.Tensor) else None


def _encode(code, inputs, dims, dtype_wire, params) -> bytes:
    out = struct.pack("<BB", code, len(inputs)) + struct.pack(f"<{len(inputs)}H", *inputs)
    out += struct.pack("<B", len(dims)) + struct.pack(f"<{len(dims)}Q", *dims)
    out += struct.pack("<BB", dtype_wire, len(params)) + struct.pack(f"<{len(params)}f", *params)
    return out


def _lower(node, index):
    """(op code, input node indices, params, output dims) of one call_function
    node, or _Unsupported.  Arguments the op list cannot carry (alpha/beta
    other than 1, several reduction dims, scalar operands other than mul's)
    make the graph unsupported rather than computing something else."""
    tgt, args, kw = node.target, node.args, node.kwargs

    def idx(a):
        if not isinstance(a, torch.fx.Node) or a.name not in index:
            raise _Unsupported(f"{tgt}: argument {a!r} is not a tensor node")
        return index[a.name]

    val = _meta(node)
    dims = list(val.shape) if val is not None else []
    if tgt in _IDENTITY_OPS:
        return OP_IDENTITY, [idx(args[0])], [], dims
    if tgt in _VIEW_OPS:
        src = _meta(args[0])
        shape = list(args[1])
        if -1 in shape:
            if src is None:
                raise _Unsupported("view with -1 of a node without shape metadata")
            known = 1
            for s in shape:
                if s != -1:
                    known *= s
            shape[shape.index(-1)] = src.numel() // max(known, 1)
        return OP_VIEW, [idx(args[0])], [], [int(s) for s in shape]
    if tgt == aten.mul.Scalar or (tgt == aten.mul.Tensor and not isinstance(args[1], torch.fx.Node)):
        return OP_SCALAR_MUL, [idx(args[0])], [float(args[1])], dims
    if tgt == aten.sum.dim_IntList:
        dim_list = args[1]
        if dim_list is None or len(dim_list) != 1 or kw.get("dtype") is not None:
            raise _Unsupported("sum over several dims")
        keep = args[2] if len(args) > 2 else kw.get("keepdim", False)
        return OP_SUM_DIM, [idx(args[0])], [float(dim_list[0]), 1.0 if keep else 0.0], dims
    if tgt not in _TENSOR_OPS:
        raise _Unsupported(f"no op code for {tgt}")
    code, n = _TENSOR_OPS[tgt]
    if kw.get("alpha", 1) != 1 or kw.get("beta", 1) != 1 or (code == OP_MEAN_ALL and kw.get("dtype") is not None):
        raise _Unsupported(f"{tgt} with {dict(kw)}")
    ins = [idx(a) for a in args[:n]]
    params = []
    if code == OP_THRESHOLD_BACKWARD:
        params = [float(args[2]) if len(args) > 2 else 0.0]
    return code, ins, params, dims


def serialize_graph(gm: torch.fx.GraphModule):
    """(op list bytes, number of placeholders, output node indices with
    NONE_OUTPUT for None) of an aot FX graph, or None when some node has no
    op code (compile_backend.py:803-903 writes the same format)."""
    index, ops, n_ph, outs = {}, bytearray(), 0, []
    try:
        for node in gm.graph.nodes:
            if node.op == "placeholder":
                index[node.name] = n_ph
                n_ph += 1
            elif node.op == "call_function":
                code, ins, params, dims = _lower(node, index)
                val = _meta(node)
                ops += _encode(code, ins, dims, _WIRE.get(val.dtype, 0) if val is not None else 0, params)
                index[node.name] = len(index)  # placeholders come first, one node per op
            elif node.op == "output":
                res = node.args[0]
                for a in (res if isinstance(res, (tuple, list)) else [res]):
                    if a is None:
                        outs.append(NONE_OUTPUT)
                    elif isinstance(a, torch.fx.Node) and a.name in index:
                        outs.append(index[a.name])
                    else:
                        raise _Unsupported(f"output {a!r}")
            else:
                raise _Unsupported(node.op)
    except _Unsupported:
        return None
    return bytes(ops), n_ph, outs


def _lib():
    from ._native import lib
    return lib


class CompiledGraphRunner:
    """Runs one aot graph: a single applegpu_eager_execute_graph call per
    invocation when the graph serializes (compile_backend.py:924-1071), the
    graph module itself on the device otherwise."""

    def __init__(self, gm: torch.fx.GraphModule):
        self.gm = gm
        ser = serialize_graph(gm)
        self.serialized = ser is not None
        if not self.serialized:
            return
        self._ops, self._n_ph, self._outs = ser
        self._ops_buf = ctypes.create_string_buffer(self._ops, len(self._ops))
        real = [i for i in self._outs if i != NONE_OUTPUT]
        self._n_real = len(real)
        self._out_idx = (ctypes.c_uint16 * max(len(real), 1))(*real)
        self._out_ids = (ctypes.c_uint64 * max(len(real), 1))()
        self._out_ptrs = (ctypes.c_void_p * max(len(real), 1))()
        self._in_ids = (ctypes.c_uint64 * max(self._n_ph, 1))()
        # output shapes as the graph declares them (a mean is 0-D here and
        # [1] on the runtime)
        self._shapes = []
        for node in gm.graph.nodes:
            if node.op == "output":
                res = node.args[0]
                for a in (res if isinstance(res, (tuple, list)) else [res]):
                    if a is not None:
                        v = _meta(a)
                        self._shapes.append(tuple(v.shape) if v is not None else None)
        self._single = not isinstance(next(n for n in gm.graph.nodes if n.op == "output").args[0], (tuple, list))

    def __call__(self, *args):
        if not self.serialized:
            return self.gm(*args)
        lib = _lib()
        views = []
        try:
            for i in range(self._n_ph):
                self._in_ids[i] = self._input_id(lib, args[i], i, views) if i < len(args) else 0
            rc = lib.applegpu_eager_execute_graph(
                ctypes.cast(self._ops_buf, ctypes.c_void_p), len(self._ops), self._in_ids, self._n_ph,
                self._out_idx, self._n_real, self._out_ids, ctypes.cast(self._out_ptrs, ctypes.POINTER(ctypes.c_void_p)))
            if rc < 0:
                err = lib.applegpu_eager_last_error()
                raise RuntimeError(err.decode() if err else "compiled graph execution failed")
            by_view = {vid: args[i] for i, vid in views}
            made = {}
            real = []
            for j in range(self._n_real):
                oid = int(self._out_ids[j])
                if oid in by_view:           # an input returned as it is
                    t = by_view[oid]
                elif oid in made:            # the same node in two output slots
                    t = made[oid]
                else:
                    t = made[oid] = torch.ops.applegpu.wrap_eager(oid)
                shape = self._shapes[j]
                if shape is not None and tuple(t.shape) != shape:
                    t = t.view(shape)
                real.append(t)
        finally:
            for _, vid in views:
                lib.applegpu_eager_free(vid)
        if self._single and len(self._outs) == 1:
            return real[0] if self._outs[0] != NONE_OUTPUT else None
        it = iter(real)
        return tuple(None if o == NONE_OUTPUT else next(it) for o in self._outs)

    @staticmethod
    def _input_id(lib, t, i, views):
        """A typed runtime view of an `applegpu` tensor (its storage's id,
        dtype, byte offset and strides), freed after the call; 0 for anything
        else (compile_backend.py:161-225 resolves ids the same way)."""
        if not isinstance(t, torch.Tensor) or t.device.type not in ("applegpu", "privateuseone"):
            return 0
        base = lib.applegpu_eager_find_by_data_ptr(ctypes.c_void_p(t.untyped_storage().data_ptr()))
        if not base:
            raise RuntimeError("applegpu tensor whose storage the runtime does not know")
        nd = max(t.dim(), 1)
        shape = (ctypes.c_uint64 * nd)(*([int(s) for s in t.shape] or [1]))
        strides = (ctypes.c_uint64 * nd)(*([int(s) for s in t.stride()] or [1]))
        vid = ctypes.c_uint64(0)
        p = lib.applegpu_eager_view_typed(base, shape, strides, nd, t.storage_offset() * t.element_size(),
                                          _WIRE[t.dtype], ctypes.byref(vid))
        if not p and not vid.value:
            err = lib.applegpu_eager_last_error()
            raise RuntimeError(err.decode() if err else "view failed")
        views.append((i, vid.value))
        return vid.value


def _compiler(gm, example_inputs):
    from torch._functorch.aot_autograd import make_boxed_func
    runner = CompiledGraphRunner(gm)
    return make_boxed_func(runner)


def applegpu_compile_backend(gm, example_inputs):
    """torch.compile backend (compile_backend.py:1085-1092): aot_autograd with
    the op-list compiler for the forward and the backward graph."""
    from torch._functorch.aot_autograd import aot_module_simplified

    from .cpp_backend import load_cpp_backend
    load_cpp_backend()
    return aot_module_simplified(gm, example_inputs, fw_compiler=_compiler, bw_compiler=_compiler)
