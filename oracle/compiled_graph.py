"""numpy restatement of the reference's torch.compile bytecode executor (test
infrastructure only: tests decode op lists with it and run them on the CPU
to check the serializer and the device executor).

Wire format, per op, little-endian (crates/core/src/compiled_graph.rs:7-9,
85-110): op_code u8, n_inputs u8, inputs u16[n], out_ndim u8,
out_dims u64[ndim], out_dtype u8, params_len u8, params f32[plen].  Node
i < n_inputs is graph input i; every op appends one node (identity appends
its input again).  Op semantics: compiled_graph.rs:122-185.

Where the reference rejects or mis-handles an input, this follows torch's
aten op instead, as the device executor does: `t` of a 0-D/1-D node is the
node (the reference errors, :168) and `view` reshapes by element order (the
reference reinterprets raw memory of non-contiguous nodes, :176-181).

Parity pins (tests/test_compile_backend.py): the decoder is checked
against hand-assembled bytes, and running op lists serialized from torch FX
graphs (an MLP's forward and its aot backward) reproduces torch CPU's own
outputs, so a swapped operand, dropped term or wrong sign fails there.
"""
from __future__ import annotations

import struct

import numpy as np

from . import ops as O

ADD, SUB, MUL, DIV, MATMUL, RELU, NEG, THRESHOLD_BACKWARD, SCALAR_MUL, MEAN_ALL, SUM_DIM, TRANSPOSE, VIEW, ADDMM = \
    range(14)
IDENTITY = 255


def decode(data: bytes) -> list[dict]:
    """Op records {code, inputs, dims, dtype, params} (compiled_graph.rs:85-110)."""
    ops, pos = [], 0

    def take(fmt):
        nonlocal pos
        size = struct.calcsize(fmt)
        if pos + size > len(data):
            raise ValueError(f"op list truncated at byte {pos}")
        vals = struct.unpack_from(fmt, data, pos)
        pos += size
        return vals

    while pos < len(data):
        code, n = take("<BB")
        inputs = list(take(f"<{n}H")) if n else []
        (nd,) = take("<B")
        dims = list(take(f"<{nd}Q")) if nd else []
        dtype, npar = take("<BB")
        params = list(take(f"<{npar}f")) if npar else []
        ops.append({"code": code, "inputs": inputs, "dims": dims, "dtype": dtype, "params": params})
    return ops


def run(data: bytes, inputs: list, output_indices: list[int]) -> list[np.ndarray]:
    """Executes the op list on numpy arrays (compiled_graph.rs:61-193)."""
    nodes = [None if x is None else np.asarray(x) for x in inputs]
    for op in decode(data):
        code, p = op["code"], op["params"]
        a = [nodes[i] for i in op["inputs"]]
        if code == IDENTITY:
            r = a[0]
        elif code in (ADD, SUB, MUL, DIV):
            r = O.broadcast_binary(("add", "sub", "mul", "div")[code], a[0], a[1]).astype(np.float32)
        elif code == MATMUL:
            r = O.matmul(a[0], a[1])
        elif code == ADDMM:
            r = (O.matmul(a[1], a[2]).astype(np.float64) + a[0]).astype(np.float32)
        elif code == RELU:
            r = O.relu(a[0])
        elif code == NEG:
            r = -a[0]
        elif code == THRESHOLD_BACKWARD:
            r = O.threshold_backward(a[0], a[1], p[0] if p else 0.0)
        elif code == SCALAR_MUL:
            r = (a[0] * np.float32(p[0] if p else 1.0)).astype(a[0].dtype)
        elif code == MEAN_ALL:
            r = O.mean_all(a[0])
        elif code == SUM_DIM:
            dim = int(p[0]) if p else 0
            r = O.sum_dim(a[0], dim, len(p) > 1 and p[1] != 0.0)
        elif code == TRANSPOSE:
            r = a[0] if a[0].ndim < 2 else np.swapaxes(a[0], -1, -2)
        elif code == VIEW:
            r = np.reshape(a[0], op["dims"])
        else:
            raise ValueError(f"unsupported op: {code}")
        nodes.append(r)
    return [nodes[i] for i in output_indices]
