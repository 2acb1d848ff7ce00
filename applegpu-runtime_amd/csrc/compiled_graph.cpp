// torch.compile bytecode executor: one C-ABI call runs a whole serialized FX
// graph (applegpu_eager_execute_graph).
//
// Wire format, per op, little-endian (crates/core/src/compiled_graph.rs:7-9,
// written by python/applegpu_runtime/compile_backend.py:803-903):
//   op_code u8, n_inputs u8, inputs u16[n], out_ndim u8, out_dims u64[ndim],
//   out_dtype u8, params_len u8, params f32[plen]
// Node i < n_inputs is graph input i; every op appends one node.  Op codes
// are the reference's (compiled_graph.rs:43-57).
//
// The reference dispatches each op to its eager runtime as it reads it
// (compiled_graph.rs:61-193).  Here every op is recorded into the lazy graph
// and all outputs are materialised by one fusion-planned walk: addmm becomes
// one GEMM with the bias (and a following relu) in its epilogue, shared
// nodes run once, and intermediates nobody returns never get an id.
// Differences from the reference, all on inputs it gets wrong or rejects:
//   - mm/addmm read strided (transposed) operands in place instead of
//     copying them contiguous first (same values);
//   - view of a non-contiguous node reshapes through a copy (the reference
//     reinterprets the raw memory, compiled_graph.rs:176-181);
//   - t of a 0-D or 1-D node is the node itself, as aten.t defines it (the
//     reference errors, compiled_graph.rs:168);
//   - a truncated or inconsistent op list is an error, not a panic.
#include <cstring>
#include <unordered_map>

#include "graph.hpp"

namespace agpu {
namespace {

enum : uint8_t {
  BC_ADD = 0, BC_SUB = 1, BC_MUL = 2, BC_DIV = 3, BC_MATMUL = 4, BC_RELU = 5, BC_NEG = 6,
  BC_THRESHOLD_BACKWARD = 7, BC_SCALAR_MUL = 8, BC_MEAN_ALL = 9, BC_SUM_DIM = 10, BC_TRANSPOSE = 11,
  BC_VIEW = 12, BC_ADDMM = 13, BC_IDENTITY = 255,
};

struct BcOp {
  uint8_t code = 0;
  std::vector<uint16_t> in;
  std::vector<int64_t> dims;
  std::vector<float> params;
};

struct Reader {
  const uint8_t* p;
  size_t n, pos = 0;
  void need(size_t k, size_t op) {
    if (n - pos < k) fail("op list truncated in op %zu (byte %zu of %zu)", op, pos, n);
  }
  template <typename T>
  T get(size_t op) {
    need(sizeof(T), op);
    T v;
    std::memcpy(&v, p + pos, sizeof(T));  // little-endian host, as the format
    pos += sizeof(T);
    return v;
  }
};

// Whole op list, checked before anything runs: every input index names an
// earlier node.
std::vector<BcOp> parse(const uint8_t* data, size_t len, uint32_t n_in) {
  if (len && !data) fail("null op list");
  std::vector<BcOp> ops;
  Reader r{data, len};
  while (r.pos < len) {
    const size_t k = ops.size();
    BcOp op;
    op.code = r.get<uint8_t>(k);
    const int ni = r.get<uint8_t>(k);
    for (int i = 0; i < ni; ++i) {
      const uint16_t idx = r.get<uint16_t>(k);
      if (idx >= n_in + k) fail("op %zu reads node %u, only %zu exist before it", k, idx, n_in + k);
      op.in.push_back(idx);
    }
    const int nd = r.get<uint8_t>(k);
    if (nd > kMaxDims) fail("op %zu: %d output dims, maximum is %d", k, nd, kMaxDims);
    for (int i = 0; i < nd; ++i) {
      const uint64_t d = r.get<uint64_t>(k);
      if (d > (uint64_t)INT64_MAX) fail("op %zu: output dim %d out of range", k, i);
      op.dims.push_back((int64_t)d);
    }
    (void)r.get<uint8_t>(k);  // output dtype: not used, as in the reference
    const int np = r.get<uint8_t>(k);
    for (int i = 0; i < np; ++i) op.params.push_back(r.get<float>(k));
    ops.push_back(std::move(op));
  }
  if (n_in + ops.size() > 0xFFFFu) fail("graph has %zu nodes; u16 indices address at most 65535", n_in + ops.size());
  return ops;
}

size_t arity(uint8_t code) {
  switch (code) {
    case BC_ADD: case BC_SUB: case BC_MUL: case BC_DIV: case BC_MATMUL: case BC_THRESHOLD_BACKWARD: return 2;
    case BC_ADDMM: return 3;
    case BC_RELU: case BC_NEG: case BC_SCALAR_MUL: case BC_MEAN_ALL: case BC_SUM_DIM: case BC_TRANSPOSE:
    case BC_VIEW: case BC_IDENTITY: return 1;
    default: fail("unsupported op: %u", (unsigned)code);
  }
}

TensorP rec(const char* name, std::vector<TensorP> in, std::vector<double> f = {}, std::vector<int64_t> iv = {}) {
  return record_op(op_code(name), in, f, iv)[0];
}

}  // namespace

void execute_compiled(const uint8_t* data, size_t len, const uint64_t* inputs, uint32_t n_in, const uint16_t* out_idx,
                      uint32_t n_out, uint64_t* out_ids, uint8_t** out_ptrs) {
  if (n_in && !inputs) fail("null input id array");
  if (n_out && (!out_idx || !out_ids || !out_ptrs)) fail("null output array");
  const std::vector<BcOp> ops = parse(data, len, n_in);
  for (size_t k = 0; k < ops.size(); ++k)
    if (ops[k].in.size() < arity(ops[k].code))
      fail("op %zu (code %u) has %zu inputs, needs %zu", k, (unsigned)ops[k].code, ops[k].in.size(),
           arity(ops[k].code));
  for (uint32_t i = 0; i < n_out; ++i)
    if (out_idx[i] >= n_in + ops.size()) fail("output %u out of range", (unsigned)out_idx[i]);

  // node -> (input id, tensor); id != 0 marks a graph input (or an identity
  // of one), returned to the caller as its own id
  struct Entry {
    uint64_t id = 0;
    TensorP t;
  };
  if (!Runtime::initialized()) fail("no device: the runtime is not initialised");
  std::vector<Entry> nodes(n_in + ops.size());
  for (uint32_t i = 0; i < n_in; ++i) nodes[i].id = inputs[i];
  Runtime& rt = Runtime::get();
  auto at = [&](uint16_t idx) -> TensorP {
    Entry& e = nodes[idx];
    if (!e.t) {
      if (!e.id) fail("graph input %u is not a device tensor", (unsigned)idx);
      e.t = rt.lookup(e.id);
    }
    return e.t;
  };

  for (size_t k = 0; k < ops.size(); ++k) {
    const BcOp& op = ops[k];
    Entry& out = nodes[n_in + k];
    auto in = [&](int i) { return at(op.in[i]); };
    const float p0 = op.params.empty() ? 0.f : op.params[0];
    switch (op.code) {
      case BC_IDENTITY: out = nodes[op.in[0]]; continue;
      case BC_ADD: out.t = rec("add", {in(0), in(1)}); break;
      case BC_SUB: out.t = rec("sub", {in(0), in(1)}); break;
      case BC_MUL: out.t = rec("mul", {in(0), in(1)}); break;
      case BC_DIV: out.t = rec("div", {in(0), in(1)}); break;
      case BC_MATMUL: out.t = rec("matmul", {in(0), in(1)}); break;
      case BC_ADDMM: {
        // bias + m1 @ m2 (alpha = beta = 1, as the serializer emits it)
        TensorP bias = in(0), mm = rec("matmul", {in(1), in(2)});
        const bool row_bias = mm->ndim == 2 && bias->ndim == 1 && bias->shape[0] == mm->shape[1];
        out.t = row_bias ? rec("add_bias", {mm, bias}) : rec("add", {mm, bias});
        break;
      }
      case BC_RELU: out.t = rec("relu", {in(0)}); break;
      case BC_NEG: out.t = rec("neg", {in(0)}); break;
      case BC_THRESHOLD_BACKWARD: out.t = rec("threshold_backward", {in(0), in(1)}, {p0}); break;
      case BC_SCALAR_MUL: out.t = rec("scalar_mul", {in(0)}, {op.params.empty() ? 1.f : p0}); break;
      case BC_MEAN_ALL: out.t = rec("mean_all", {in(0)}); break;
      case BC_SUM_DIM: {
        const bool keep = op.params.size() > 1 && op.params[1] != 0.f;
        out.t = rec("sum_dim", {in(0)}, {}, {(int64_t)p0, keep ? 1 : 0});
        break;
      }
      case BC_TRANSPOSE: {
        TensorP x = in(0);
        out.t = x->ndim < 2 ? x : rec("transpose", {x});
        if (x->ndim < 2) out.id = nodes[op.in[0]].id;
        break;
      }
      case BC_VIEW: out.t = rec("reshape", {in(0)}, {}, op.dims); break;
      default: fail("unsupported op: %u", (unsigned)op.code);
    }
  }

  // Keep the returned nodes; drop every other reference so single-use
  // intermediates can fuse into their consumers.
  std::vector<TensorP> roots;
  std::vector<Entry> outs(n_out);
  for (uint32_t i = 0; i < n_out; ++i) {
    outs[i] = nodes[out_idx[i]];
    if (!outs[i].t && outs[i].id) outs[i].t = rt.lookup(outs[i].id);
    if (!outs[i].t) fail("output %u is graph input %u, which is not a device tensor", i, (unsigned)out_idx[i]);
    roots.push_back(outs[i].t);
  }
  nodes.clear();
  eval_all(roots);

  std::unordered_map<Tensor*, uint64_t> given;
  for (uint32_t i = 0; i < n_out; ++i) {
    uint64_t id = outs[i].id;
    if (!id) {
      auto it = given.find(outs[i].t.get());
      id = it != given.end() ? it->second : (given[outs[i].t.get()] = rt.insert(outs[i].t));
    }
    out_ids[i] = id;
    out_ptrs[i] = (uint8_t*)outs[i].t->data();
  }
}

}  // namespace agpu
