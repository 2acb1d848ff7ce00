// Op layer: validation (the reference's dtype/shape rules), layouts, launches.
//
// Reference rules followed (crates/core/src/ops.rs unless noted):
//   dtype classes per op              :29-170 (validate_op_dtype)
//   binary: same dtype, broadcast     :172-202; comparisons -> bool :222-246
//   matmul: >=2-D, inner dims match, batch dims broadcast            :390-462
//   softmax / log_softmax >=1-D       :464-508; softmax_causal >=2-D :1367-1388
//   layer_norm gamma/beta shape [C]   :618-653
//   embedding: W 2-D, int32 indices   :1194-1232
//   slice / concat / add_bias         :1234-1365
//   argmax -> int32, [...,C] -> [...] (1-D -> [1])                   :1390-1415
//   gather / index_select             :1729-1835
//   quantize / dequantize             :2250-2297
//   sum_dim output shape              crates/core/src/eager.rs:827-855
#include "ops.hpp"
#include "graph.hpp"

#include <cmath>

namespace agpu {
namespace ops {

static Runtime& rt() { return Runtime::get(); }

// In meta mode (lazy recording) outputs are descriptions without storage and
// nothing is launched.
static TensorP alloc_out(DType dt, const std::vector<int64_t>& dims) {
  if (meta_mode()) return make_meta(dt, dims);
  return rt().alloc(dt, dims);
}
static BufferP scratch(size_t bytes) {
  if (meta_mode()) return nullptr;
  return rt().pool().acquire(bytes);
}
// Kernel launches are skipped while ops only infer shapes.  Written as
// if-else so that an `else` after `if (c) LAUNCH f();` binds to `if (c)`.
#define LAUNCH if (meta_mode()) {} else

// ── dtype rules ────────────────────────────────────────────────────────────
enum Cls { kFloatOnly, kNumeric, kAny, kNotBool, kOrdered, kEquality, kIntOrBool, kIntOnly };

static void check_dtype(const char* op, Cls c, DType d) {
  if (d == DType::F64) fail("%s: float64 is not supported on this device path", op);
  bool ok = true;
  switch (c) {
    case kFloatOnly: ok = dtype_is_float(d); break;
    case kNumeric: ok = !(d == DType::Bool || d == DType::I8 || d == DType::I16); break;
    case kAny: ok = true; break;
    case kNotBool: ok = d != DType::Bool; break;
    case kOrdered:
      ok = dtype_is_float(d) || d == DType::I32 || d == DType::I64 || d == DType::U8 || d == DType::U32;
      break;
    case kEquality:
      ok = dtype_is_float(d) || d == DType::I32 || d == DType::I64 || d == DType::U8 || d == DType::U32 ||
           d == DType::Bool;
      break;
    case kIntOrBool:
      ok = d == DType::I32 || d == DType::I64 || d == DType::U8 || d == DType::U32 || d == DType::Bool;
      break;
    case kIntOnly: ok = d == DType::I32 || d == DType::I64 || d == DType::U8 || d == DType::U32; break;
  }
  static const char* kWant[] = {"a float dtype", "a numeric dtype", "any dtype", "a non-bool dtype",
                                "an ordered dtype", "a comparable dtype", "an integer or bool dtype",
                                "an integer dtype"};
  if (!ok) fail("%s does not support dtype %s (needs %s)", op, dtype_name(d), kWant[(int)c]);
}

static const char* bin_name(int op) {
  static const char* n[] = {"add", "sub", "mul", "div", "elem_min", "elem_max", "mod", "bitwise_and",
                            "bitwise_or", "bitwise_xor", "lt", "gt", "le", "ge", "eq", "ne",
                            "threshold_backward", "softmax_backward", "gelu_backward", "gelu_exact_backward"};
  return op >= 0 && op <= k::kGeluExactBwd ? n[op] : "binary";
}

static Cls bin_class(int op) {
  switch (op) {
    case k::kAdd: case k::kSub: case k::kMul: case k::kDiv: return kNumeric;
    case k::kMin: case k::kMax: case k::kMod: return kNumeric;
    case k::kAnd: case k::kOr: case k::kXor: return kIntOrBool;
    case k::kLt: case k::kGt: case k::kLe: case k::kGe: return kOrdered;
    case k::kEq: case k::kNe: return kEquality;
    case k::kThresholdBwd: case k::kGeluBwd: case k::kGeluExactBwd: return kFloatOnly;
  }
  return kAny;
}

// ── layouts ────────────────────────────────────────────────────────────────
k::ND nd_shape(const std::vector<int64_t>& dims) {
  k::ND s;
  s.ndim = (int)dims.size();
  int64_t st = 1;
  for (int i = s.ndim - 1; i >= 0; --i) {
    s.shape[i] = dims[i];
    s.stride[i] = st;
    st *= dims[i];
  }
  return s;
}

k::ND nd_for(const Tensor& t, const std::vector<int64_t>& out) {
  k::ND s;
  s.ndim = (int)out.size();
  const int off = s.ndim - t.ndim;
  if (off < 0) fail("internal: operand has more dims than the output");
  for (int i = 0; i < s.ndim; ++i) {
    s.shape[i] = out[i];
    if (i < off) { s.stride[i] = 0; continue; }
    const int ti = i - off;
    s.stride[i] = (t.shape[ti] == out[i] && t.shape[ti] != 1) ? t.strides[ti] : 0;
  }
  return s;
}

static TensorP materialize(const TensorP& t) {
  TensorP out = alloc_out(t->dtype, t->dims());
  auto dims = t->dims();
  LAUNCH k::unary(k::kCopy, t->dtype, t->dtype, t->data(), nd_for(*t, dims), out->data(), nd_shape(dims), 0, 0,
           rt().stream());
  return out;
}

TensorP contiguous(const TensorP& t) {
  if (meta_mode()) return t->is_contiguous() ? t : make_meta(t->dtype, t->dims());
  if (t->pending()) fail("internal: tensor still pending");
  if (t->is_contiguous()) return t;
  return materialize(t);
}

bool as_rows(const Tensor& t, int64_t* rows, int64_t* ld) {
  if (t.ndim == 0) { *rows = 1; *ld = 1; return true; }
  const int64_t cols = t.shape[t.ndim - 1];
  if (cols > 1 && t.strides[t.ndim - 1] != 1) return false;
  int64_t r = 1;
  for (int i = 0; i < t.ndim - 1; ++i) r *= t.shape[i];
  // leading dims must collapse to a single row stride
  int64_t stride = -1;
  int64_t expect_inner = -1;
  for (int i = t.ndim - 2; i >= 0; --i) {
    if (t.shape[i] == 1) continue;
    if (stride < 0) {
      stride = t.strides[i];
      expect_inner = stride * t.shape[i];
    } else {
      if (t.strides[i] != expect_inner) return false;
      expect_inner *= t.shape[i];
    }
  }
  if (stride < 0) stride = cols;
  if (r > 1 && stride < cols) return false;
  *rows = r;
  *ld = stride;
  return true;
}

TensorP view_bytes(const TensorP& base, DType dt, const std::vector<int64_t>& shape,
                   const std::vector<int64_t>& strides, int64_t offset_bytes) {
  if (shape.size() != strides.size()) fail("view: shape and strides differ in length");
  if (!base->buf) fail("view: base tensor has no storage");
  if (offset_bytes < 0) fail("view: negative byte offset");
  auto t = make_meta(dt, shape);
  for (size_t i = 0; i < shape.size(); ++i) {
    if (strides[i] < 0) fail("view: negative strides are not supported");
    t->strides[i] = strides[i];
  }
  t->buf = base->buf;
  t->offset = base->offset + offset_bytes;
  if ((size_t)t->offset + t->extent_bytes() > base->buf->requested)
    fail("view: shape %s (%s) with the given strides and byte offset exceeds the base storage",
         shape_str(shape).c_str(), dtype_name(dt));
  return t;
}

TensorP view(const TensorP& base, const std::vector<int64_t>& shape, const std::vector<int64_t>& strides,
             int64_t offset_elems) {
  if (shape.size() != strides.size()) fail("view: shape and strides differ in length");
  auto t = make_meta(base->dtype, shape);
  for (size_t i = 0; i < shape.size(); ++i) t->strides[i] = strides[i];
  t->buf = base->buf;
  t->offset = base->offset + offset_elems * (int64_t)dtype_size(base->dtype);
  // Bounds: the view must stay inside the base allocation.
  int64_t last = 0;
  for (size_t i = 0; i < shape.size(); ++i) {
    if (shape[i] == 0) { last = -1; break; }
    if (strides[i] < 0) fail("view: negative strides are not supported");
    last += (shape[i] - 1) * strides[i];
  }
  if (base->buf && last >= 0 &&
      (size_t)(t->offset + (last + 1) * (int64_t)dtype_size(base->dtype)) > base->buf->requested)
    fail("view: shape %s with the given strides/offset exceeds the base storage", shape_str(shape).c_str());
  return t;
}

TensorP reshape(const TensorP& t, const std::vector<int64_t>& shape) {
  int64_t n = 1;
  for (auto d : shape) n *= d;
  if (n != t->numel())
    fail("Cannot reshape: old shape %s has %lld elements, new shape %s has %lld",
         shape_str(t->dims()).c_str(), (long long)t->numel(), shape_str(shape).c_str(), (long long)n);
  TensorP src = t;
  // Try to express the new shape as a view: split/merge dims only inside
  // runs that are contiguous with each other.
  std::vector<int64_t> nstr(shape.size());
  {
    int oi = src->ndim - 1, ni = (int)shape.size() - 1;
    bool ok = true;
    while (ok && (oi >= 0 || ni >= 0)) {
      // skip size-1 dims
      if (ni >= 0 && shape[ni] == 1) { nstr[ni] = ni + 1 < (int)shape.size() ? nstr[ni + 1] * shape[ni + 1] : 1; --ni; continue; }
      if (oi >= 0 && src->shape[oi] == 1) { --oi; continue; }
      if (oi < 0 || ni < 0) { ok = false; break; }
      // gather a group of old dims and new dims with equal products
      int64_t op = src->shape[oi], np = shape[ni];
      int o_lo = oi, n_lo = ni;
      while (op != np) {
        if (op < np) { if (--o_lo < 0) { ok = false; break; } op *= src->shape[o_lo]; }
        else { if (--n_lo < 0) { ok = false; break; } np *= shape[n_lo]; }
      }
      if (!ok) break;
      // old dims o_lo..oi must be mutually contiguous (ignoring size-1 dims)
      int64_t inner_stride = src->strides[oi];
      int64_t expect = inner_stride;
      for (int j = oi; j >= o_lo; --j) {
        if (src->shape[j] == 1) continue;
        if (src->strides[j] != expect) { ok = false; break; }
        expect *= src->shape[j];
      }
      if (!ok) break;
      int64_t s = inner_stride;
      for (int j = ni; j >= n_lo; --j) {
        nstr[j] = s;
        s *= shape[j];
      }
      oi = o_lo - 1;
      ni = n_lo - 1;
    }
    if (ok && !src->pending()) {
      auto v = make_meta(src->dtype, shape);
      for (size_t i = 0; i < shape.size(); ++i) v->strides[i] = nstr[i];
      v->buf = src->buf;
      v->offset = src->offset;
      return v;
    }
  }
  TensorP c = materialize(src);
  auto v = make_meta(c->dtype, shape);
  v->buf = c->buf;
  v->offset = c->offset;
  return v;
}

TensorP transpose_dims(const TensorP& t, int d0, int d1) {
  if (d0 < 0 || d1 < 0 || d0 >= t->ndim || d1 >= t->ndim)
    fail("transpose dims (%d, %d) out of range for %dD tensor", d0, d1, t->ndim);
  auto v = std::make_shared<Tensor>(*t);
  v->node = nullptr;
  v->ext_refs = 0;
  std::swap(v->shape[d0], v->shape[d1]);
  std::swap(v->strides[d0], v->strides[d1]);
  return v;
}

TensorP slice(const TensorP& t, int dim, int64_t start, int64_t end) {
  if (dim < 0 || dim >= t->ndim) fail("slice dim %d >= ndim %d", dim, t->ndim);
  if (start >= end) fail("slice start %lld >= end %lld", (long long)start, (long long)end);
  if (end > t->shape[dim]) fail("slice end %lld > shape[%d] = %lld", (long long)end, dim, (long long)t->shape[dim]);
  auto v = std::make_shared<Tensor>(*t);
  v->node = nullptr;
  v->ext_refs = 0;
  v->shape[dim] = end - start;
  v->offset = t->offset + start * t->strides[dim] * (int64_t)dtype_size(t->dtype);
  return v;
}

// ── elementwise ────────────────────────────────────────────────────────────
TensorP binary(int op, const TensorP& a, const TensorP& b, float p0) {
  if (a->dtype != b->dtype) fail("Dtype mismatch: %s vs %s", dtype_name(a->dtype), dtype_name(b->dtype));
  check_dtype(bin_name(op), bin_class(op), a->dtype);
  auto out_dims = broadcast_shapes(a->dims(), b->dims());
  bool cmp = op >= k::kLt && op <= k::kNe;
  DType odt = cmp ? DType::Bool : a->dtype;
  TensorP out = alloc_out(odt, out_dims);
  LAUNCH k::binary(op, a->dtype, odt, a->data(), nd_for(*a, out_dims), b->data(), nd_for(*b, out_dims), out->data(),
            nd_shape(out_dims), p0, rt().stream());
  return out;
}

static const char* un_name(int op) {
  switch (op) {
    case k::kNeg: return "neg"; case k::kRelu: return "relu"; case k::kExp: return "exp";
    case k::kLog: return "log"; case k::kSqrt: return "sqrt"; case k::kAbs: return "abs";
    case k::kSign: return "sign"; case k::kTanh: return "tanh"; case k::kSin: return "sin";
    case k::kCos: return "cos"; case k::kSigmoid: return "sigmoid"; case k::kGelu: return "gelu";
    case k::kGeluExact: return "gelu_exact"; case k::kScale: return "scalar_mul"; case k::kPow: return "pow";
    case k::kClamp: return "clamp"; case k::kBitNot: return "bitwise_not"; case k::kLogicalNot: return "logical_not";
    case k::kShl: return "shl"; case k::kShr: return "shr"; case k::kCopy: return "copy";
  }
  return "unary";
}

static Cls un_class(int op) {
  switch (op) {
    case k::kNeg: case k::kAbs: case k::kSign: case k::kScale: case k::kClamp: return kNumeric;
    case k::kBitNot: return kIntOrBool;
    case k::kShl: case k::kShr: return kIntOnly;
    case k::kLogicalNot: case k::kCopy: return kAny;
    case k::kPow: return kFloatOnly;
  }
  return kFloatOnly;
}

TensorP fused_chain(const std::vector<TensorP>& leaves, const k::ChainProgram& prog, DType dt,
                    const std::vector<int64_t>& dims) {
  if (dt != DType::F32 && dt != DType::F16 && dt != DType::BF16) fail("fused_chain: %s is not a float dtype", dtype_name(dt));
  if (leaves.empty() || leaves.size() > (size_t)k::kChainMaxLeaves || (int)leaves.size() != prog.n_leaves)
    fail("fused_chain: %zu leaves for a program of %d", leaves.size(), prog.n_leaves);
  k::ChainLeaves L;
  for (size_t j = 0; j < leaves.size(); ++j) {
    if (leaves[j]->dtype != dt) fail("fused_chain: leaf %zu is %s, not %s", j, dtype_name(leaves[j]->dtype), dtype_name(dt));
    if (broadcast_shapes(leaves[j]->dims(), dims) != dims) fail("fused_chain: leaf %zu does not broadcast to the output", j);
  }
  TensorP out = alloc_out(dt, dims);
  LAUNCH {
    for (size_t j = 0; j < leaves.size(); ++j) {
      L.ptr[j] = leaves[j]->data();
      L.nd[j] = nd_for(*leaves[j], dims);
    }
    k::fused_chain(dt, prog, L, out->data(), nd_shape(dims), rt().stream());
  }
  return out;
}

TensorP unary(int op, const TensorP& x, float p0, float p1) {
  check_dtype(un_name(op), un_class(op), x->dtype);
  DType odt = op == k::kLogicalNot ? DType::Bool : x->dtype;
  auto dims = x->dims();
  TensorP out = alloc_out(odt, dims);
  LAUNCH k::unary(op, x->dtype, odt, x->data(), nd_for(*x, dims), out->data(), nd_shape(dims), p0, p1, rt().stream());
  return out;
}

TensorP cast(const TensorP& x, DType dt) {
  if (x->dtype == DType::F64 || dt == DType::F64) fail("cast: float64 is not supported on this device path");
  if (x->dtype == dt) return x;
  auto dims = x->dims();
  TensorP out = alloc_out(dt, dims);
  LAUNCH k::unary(k::kCopy, x->dtype, dt, x->data(), nd_for(*x, dims), out->data(), nd_shape(dims), 0, 0, rt().stream());
  return out;
}

TensorP quantize(const TensorP& x, DType dt, float scale, int zp) {
  if (!dtype_is_float(x->dtype) || x->dtype == DType::F64) fail("Quantize input must be a float dtype");
  if (dt != DType::I8 && dt != DType::U8) fail("Quantize target must be Int8 or UInt8");
  if (scale == 0.f) fail("Quantize scale must be non-zero");
  auto dims = x->dims();
  TensorP out = alloc_out(dt, dims);
  LAUNCH k::unary(k::kQuantize, x->dtype, dt, x->data(), nd_for(*x, dims), out->data(), nd_shape(dims), scale, (float)zp,
           rt().stream());
  return out;
}

TensorP dequantize(const TensorP& x, DType dt, float scale, int zp) {
  if (x->dtype != DType::I8 && x->dtype != DType::U8) fail("Dequantize input must be Int8 or UInt8");
  if (!dtype_is_float(dt) || dt == DType::F64) fail("Dequantize target must be a float dtype");
  auto dims = x->dims();
  TensorP out = alloc_out(dt, dims);
  LAUNCH k::unary(k::kDequantize, x->dtype, dt, x->data(), nd_for(*x, dims), out->data(), nd_shape(dims), scale,
           (float)zp, rt().stream());
  return out;
}

TensorP where(const TensorP& c, const TensorP& x, const TensorP& y) {
  if (x->dtype != y->dtype) fail("where: dtype mismatch %s vs %s", dtype_name(x->dtype), dtype_name(y->dtype));
  check_dtype("where", kAny, x->dtype);
  auto dims = broadcast_shapes(broadcast_shapes(c->dims(), x->dims()), y->dims());
  TensorP out = alloc_out(x->dtype, dims);
  LAUNCH k::where(c->dtype, x->dtype, c->data(), nd_for(*c, dims), x->data(), nd_for(*x, dims), y->data(),
           nd_for(*y, dims), out->data(), nd_shape(dims), rt().stream());
  return out;
}

TensorP full(DType dt, const std::vector<int64_t>& dims, float value) {
  TensorP out = alloc_out(dt, dims);
  LAUNCH k::unary(k::kFill, dt, dt, out->data(), nd_shape(dims), out->data(), nd_shape(dims), value, 0, rt().stream());
  return out;
}

TensorP masked_fill(const TensorP& x, const TensorP& mask, float value) {
  TensorP v = full(x->dtype, {1}, value);
  return where(mask, v, x);
}

TensorP tri(const TensorP& x, bool upper, int64_t diag) {
  if (x->ndim < 2) fail("%s requires at least 2D tensor", upper ? "triu" : "tril");
  TensorP c = contiguous(x);
  int64_t rows = c->shape[c->ndim - 2], cols = c->shape[c->ndim - 1];
  TensorP out = alloc_out(c->dtype, c->dims());
  LAUNCH k::tri(c->dtype, upper, diag, c->data(), out->data(), c->numel() / std::max<int64_t>(rows * cols, 1), rows,
         cols, rt().stream());
  return out;
}

TensorP threshold_backward(const TensorP& grad, const TensorP& input, float thr) {
  if (grad->dtype != input->dtype)
    fail("dtype mismatch: %s vs %s", dtype_name(grad->dtype), dtype_name(input->dtype));
  return binary(k::kThresholdBwd, grad, input, thr);
}

TensorP add_bias(const TensorP& x, const TensorP& bias) {
  check_dtype("add_bias", kFloatOnly, x->dtype);
  if (x->dtype != bias->dtype)
    fail("add_bias dtype mismatch: %s vs %s", dtype_name(x->dtype), dtype_name(bias->dtype));
  if (x->ndim < 2) fail("add_bias requires >= 2D input, got %s", shape_str(x->dims()).c_str());
  if (bias->ndim != 1) fail("add_bias requires 1D bias, got %s", shape_str(bias->dims()).c_str());
  if (bias->shape[0] != x->shape[1])
    fail("add_bias bias length %lld != input dim 1 %lld", (long long)bias->shape[0], (long long)x->shape[1]);
  TensorP c = contiguous(x);
  TensorP b = contiguous(bias);
  int64_t cs = 1;
  for (int i = 2; i < c->ndim; ++i) cs *= c->shape[i];
  TensorP out = alloc_out(c->dtype, c->dims());
  LAUNCH k::add_bias(c->dtype, c->data(), b->data(), out->data(), c->numel(), c->shape[1], cs, rt().stream());
  return out;
}

void axpy_inplace(const TensorP& self, const TensorP& other, float alpha) {
  if (!self->is_contiguous()) fail("in-place op on non-contiguous tensor not yet supported");
  if (self->dtype != other->dtype)
    fail("dtype mismatch: %s vs %s", dtype_name(self->dtype), dtype_name(other->dtype));
  check_dtype("add_scaled_inplace", kFloatOnly, self->dtype);
  auto dims = self->dims();
  broadcast_shapes(dims, other->dims());  // validates
  if (other->ndim > self->ndim) fail("in-place add: other has more dims than self");
  for (int i = 0; i < other->ndim; ++i) {
    int64_t od = other->shape[other->ndim - 1 - i], sd = self->shape[self->ndim - 1 - i];
    if (od != sd && od != 1) fail("in-place add: cannot broadcast %s onto %s", shape_str(other->dims()).c_str(),
                                  shape_str(dims).c_str());
  }
  LAUNCH k::axpy(self->dtype, self->data(), nd_shape(dims), other->data(), nd_for(*other, dims), alpha, rt().stream());
}

void copy_into(const TensorP& dst, const TensorP& src) {
  auto dims = dst->dims();
  if (src->numel() != dst->numel()) fail("copy: element counts differ (%lld vs %lld)", (long long)src->numel(),
                                         (long long)dst->numel());
  TensorP s = src;
  if (src->dims() != dims) s = reshape(src, dims);
  if (dst->is_contiguous()) {
    LAUNCH k::unary(k::kCopy, s->dtype, dst->dtype, s->data(), nd_for(*s, dims), dst->data(), nd_shape(dims), 0, 0,
             rt().stream());
    return;
  }
  // Strided destination (a slice or transpose of a larger tensor): every
  // element must have its own address.
  k::ND so;
  so.ndim = dst->ndim;
  for (int i = 0; i < dst->ndim; ++i) {
    so.shape[i] = dst->shape[i];
    so.stride[i] = dst->strides[i];
    if (dst->shape[i] > 1 && dst->strides[i] == 0)
      fail("copy: the destination has overlapping elements (stride 0 in dim %d)", i);
  }
  LAUNCH k::copy_strided(s->dtype, dst->dtype, s->data(), nd_for(*s, dims), dst->data(), so, rt().stream());
}

// ── rows ───────────────────────────────────────────────────────────────────
TensorP softmax(const TensorP& x, int mode) {
  const char* name = mode == k::kSoftmax ? "softmax" : mode == k::kLogSoftmax ? "log_softmax" : "softmax_causal";
  check_dtype(name, kFloatOnly, x->dtype);
  if (mode == k::kSoftmaxCausal) {
    if (x->ndim < 2) fail("softmax_causal requires at least 2D tensor, got %s", shape_str(x->dims()).c_str());
  } else if (x->ndim < 1) {
    fail("%s requires at least 1D tensor", name);
  }
  TensorP src = x;
  int64_t rows, ld;
  if (!as_rows(*src, &rows, &ld)) {
    src = contiguous(x);
    as_rows(*src, &rows, &ld);
  }
  const int64_t cols = x->shape[x->ndim - 1];
  TensorP out = alloc_out(x->dtype, x->dims());
  int64_t crow = mode == k::kSoftmaxCausal ? x->shape[x->ndim - 2] : rows;
  LAUNCH k::softmax_rows(mode, x->dtype, src->data(), ld, out->data(), cols, rows, cols, crow, rt().stream());
  return out;
}

TensorP layer_norm(const TensorP& x, const TensorP& g, const TensorP& b, float eps) {
  check_dtype("layer_norm", kFloatOnly, x->dtype);
  if (x->ndim < 1) fail("layer_norm requires at least 1D input");
  const int64_t cols = x->shape[x->ndim - 1];
  if (!(g->ndim == 1 && g->shape[0] == cols)) fail("gamma shape %s must be [%lld]", shape_str(g->dims()).c_str(), (long long)cols);
  if (!(b->ndim == 1 && b->shape[0] == cols)) fail("beta shape %s must be [%lld]", shape_str(b->dims()).c_str(), (long long)cols);
  if (g->dtype != x->dtype || b->dtype != x->dtype) fail("layer_norm: gamma/beta dtype must match the input");
  TensorP src = x;
  int64_t rows, ld;
  if (!as_rows(*src, &rows, &ld)) {
    src = contiguous(x);
    as_rows(*src, &rows, &ld);
  }
  TensorP gc = contiguous(g), bc = contiguous(b);
  TensorP out = alloc_out(x->dtype, x->dims());
  LAUNCH k::layer_norm(x->dtype, src->data(), ld, gc->data(), bc->data(), out->data(), rows, cols, eps, rt().stream());
  return out;
}

// Rows at least this long, when there are at most kLongRowsMax of them,
// reduce (sum, mean) over many blocks.
constexpr int64_t kLongRowCols = (int64_t)1 << 20;
constexpr int64_t kLongRowsMax = 16;

TensorP row_reduce(int op, const TensorP& x, int correction) {
  const char* name = op == k::kRSum ? "sum" : op == k::kRMean ? "mean" : op == k::kRAmax ? "amax"
                     : op == k::kRArgmax ? "argmax" : "var";
  if (op == k::kRSum || op == k::kRArgmax) check_dtype(name, kNotBool, x->dtype);
  else if (op == k::kRAmax) check_dtype(name, kNotBool, x->dtype);
  else check_dtype(name, kFloatOnly, x->dtype);
  if (x->ndim < 1) fail("%s requires at least 1D tensor", name);
  std::vector<int64_t> od(x->shape, x->shape + x->ndim - 1);
  if (od.empty()) od = {1};
  TensorP src = x;
  int64_t rows, ld;
  if (!as_rows(*src, &rows, &ld)) {
    src = contiguous(x);
    as_rows(*src, &rows, &ld);
  }
  DType odt = op == k::kRArgmax ? DType::I32 : x->dtype;
  TensorP out = alloc_out(odt, od);
  const int64_t cols = x->shape[x->ndim - 1];
  if ((op == k::kRSum || op == k::kRMean) && dtype_is_float(x->dtype) && x->dtype != DType::F64 &&
      rows <= kLongRowsMax && cols >= kLongRowCols) {
    // A few very long rows: one wavefront per row would read each at a few
    // GB/s; each row takes the two-stage all-element reduction instead (512
    // blocks of fp32 partials, then one block).
    BufferP ws = scratch(k::reduce_all_ws_bytes());
    const size_t es = dtype_size(x->dtype);
    for (int64_t r = 0; r < rows; ++r)
      LAUNCH k::reduce_all(0, x->dtype, (const char*)src->data() + r * ld * (int64_t)es, nullptr, cols,
                           op == k::kRMean ? 1.f / (float)cols : 1.f, (char*)out->data() + r * (int64_t)es, ws->ptr,
                           rt().stream());
    return out;
  }
  LAUNCH k::row_reduce(op, x->dtype, odt, src->data(), ld, out->data(), rows, cols, correction, rt().stream());
  return out;
}

TensorP softmax_backward(const TensorP& dy, const TensorP& y) {
  check_dtype("softmax_backward", kFloatOnly, dy->dtype);
  if (dy->dims() != y->dims() || dy->dtype != y->dtype) fail("softmax_backward: shape/dtype mismatch");
  TensorP a = contiguous(dy), b = contiguous(y);
  int64_t cols = a->shape[a->ndim - 1];
  TensorP out = alloc_out(a->dtype, a->dims());
  LAUNCH k::softmax_backward(a->dtype, a->data(), b->data(), out->data(), a->numel() / std::max<int64_t>(cols, 1), cols,
                      rt().stream());
  return out;
}

// layer_norm backward (ops.rs:690-728 validates the same shapes): dx, and
// with `params` also dgamma = sum_r dy * xhat and dbeta = sum_r dy, each
// formed from statistics recomputed from x, or from the forward's saved
// mean and rstd (one value per row) when given.
std::vector<TensorP> layer_norm_grads(const TensorP& dy, const TensorP& x, const TensorP& g, float eps, bool params,
                                      const TensorP& mean, const TensorP& rstd) {
  check_dtype("layer_norm_backward", kFloatOnly, dy->dtype);
  if (dy->dims() != x->dims())
    fail("layer_norm_backward: grad_output shape %s != input shape %s", shape_str(dy->dims()).c_str(),
         shape_str(x->dims()).c_str());
  if (dy->dtype != x->dtype || g->dtype != x->dtype) fail("layer_norm_backward: dtypes of grad, input and gamma differ");
  if (x->ndim < 1) fail("layer_norm_backward requires at least 1D tensor");
  const int64_t cols = x->shape[x->ndim - 1];
  if (!(g->ndim == 1 && g->shape[0] == cols))
    fail("layer_norm_backward: gamma shape %s must be [%lld]", shape_str(g->dims()).c_str(), (long long)cols);
  TensorP a = contiguous(dy), b = contiguous(x), gc = contiguous(g);
  const int64_t rows = cols ? b->numel() / cols : 0;
  TensorP mc, rc;
  if (mean || rstd) {
    if (!mean || !rstd) fail("layer_norm_backward: saved mean and rstd go together");
    if (mean->numel() != rows || rstd->numel() != rows || mean->dtype != x->dtype || rstd->dtype != x->dtype)
      fail("layer_norm_backward: saved mean/rstd must hold one %s per row (%lld rows)", dtype_name(x->dtype),
           (long long)rows);
    mc = contiguous(mean);
    rc = contiguous(rstd);
  }
  const void* mp = mc ? mc->data() : nullptr;
  const void* rp = rc ? rc->data() : nullptr;
  TensorP dx = alloc_out(x->dtype, x->dims());
  if (!params) {
    LAUNCH k::layer_norm_backward(x->dtype, a->data(), b->data(), gc->data(), dx->data(), nullptr, mp, rp, rows, cols,
                                  eps, rt().stream());
    return {dx};
  }
  TensorP dg = alloc_out(x->dtype, {cols}), db = alloc_out(x->dtype, {cols});
  if (!meta_mode()) {
    BufferP st = scratch((size_t)std::max<int64_t>(rows, 1) * 2 * sizeof(float));
    BufferP ws = scratch(std::max<size_t>(k::layer_norm_param_ws_bytes(rows, cols), 4));
    k::layer_norm_backward(x->dtype, a->data(), b->data(), gc->data(), dx->data(), (float*)st->ptr, mp, rp, rows,
                           cols, eps, rt().stream());
    k::layer_norm_param_grads(x->dtype, a->data(), b->data(), (const float*)st->ptr, dg->data(), db->data(),
                              (float*)ws->ptr, rows, cols, rt().stream());
  }
  return {dx, dg, db};
}

TensorP gelu_backward(const TensorP& grad, const TensorP& x, bool exact) {
  // ops.rs:1090-1158: same shapes and dtype; the tanh form is gelu_backward
  // and gelu_tanh_backward, the erf form gelu_exact_backward
  if (grad->dims() != x->dims())
    fail("gelu_backward shape mismatch: grad %s vs input %s", shape_str(grad->dims()).c_str(),
         shape_str(x->dims()).c_str());
  return binary(exact ? k::kGeluExactBwd : k::kGeluBwd, grad, x);
}

TensorP embedding_backward(const TensorP& grad, const TensorP& idx, int64_t num_weights) {
  // ops.rs:915-960: int indices, grad [..., D] whose leading extent is the
  // number of indices; the result is [num_weights, D] in grad's dtype
  check_dtype("embedding_backward", kFloatOnly, grad->dtype);
  if (idx->dtype != DType::I32 && idx->dtype != DType::I64)
    fail("embedding_backward indices must be Int32, got %s", dtype_name(idx->dtype));
  if (grad->ndim < 1) fail("embedding_backward grad_output must have at least 1 dimension");
  if (idx->ndim < 1) fail("embedding_backward indices must have at least 1 dimension");
  if (num_weights < 0) fail("embedding_backward: negative num_weights");
  const int64_t dim = grad->shape[grad->ndim - 1];
  const int64_t n = idx->numel();
  const int64_t prefix = dim ? grad->numel() / dim : 0;
  if (dim && prefix != n)
    fail("embedding_backward: grad_output prefix %lld != indices numel %lld", (long long)prefix, (long long)n);
  TensorP gc = contiguous(grad), ic = contiguous(idx);
  TensorP out = alloc_out(grad->dtype, {num_weights, dim});
  LAUNCH k::embedding_backward(grad->dtype, gc->data(), ic->dtype, ic->data(), n, dim, num_weights, out->data(),
                               rt().stream());
  return out;
}

std::pair<TensorP, TensorP> quantize_per_row(const TensorP& x) {
  check_dtype("quantize_per_row", kFloatOnly, x->dtype);
  if (x->ndim < 1) fail("quantize_per_row requires at least 1D input");
  TensorP c = contiguous(x);
  int64_t cols = c->shape[c->ndim - 1];
  int64_t rows = cols ? c->numel() / cols : 0;
  std::vector<int64_t> sd(c->shape, c->shape + c->ndim - 1);
  if (sd.empty()) sd = {1};
  TensorP q = alloc_out(DType::I8, c->dims());
  TensorP s = alloc_out(DType::F32, sd);
  LAUNCH k::quantize_rows(c->dtype, c->data(), (int8_t*)q->data(), (float*)s->data(), rows, cols, rt().stream());
  return {q, s};
}

TensorP dequantize_per_row(const TensorP& q, const TensorP& scale, DType dt) {
  if (q->dtype != DType::I8) fail("dequantize_per_row: codes must be int8");
  if (scale->dtype != DType::F32) fail("dequantize_per_row: scales must be float32");
  if (!dtype_is_float(dt) || dt == DType::F64) fail("dequantize_per_row: target must be a float dtype");
  TensorP qc = contiguous(q), sc = contiguous(scale);
  int64_t cols = qc->shape[qc->ndim - 1];
  int64_t rows = cols ? qc->numel() / cols : 0;
  if (sc->numel() != rows) fail("dequantize_per_row: %lld scales for %lld rows", (long long)sc->numel(), (long long)rows);
  TensorP out = alloc_out(dt, qc->dims());
  LAUNCH k::dequantize_rows(dt, (const int8_t*)qc->data(), (const float*)sc->data(), out->data(), rows, cols, rt().stream());
  return out;
}

// ── reductions ─────────────────────────────────────────────────────────────
TensorP sum_dim(const TensorP& x, int64_t dim, bool keepdim, float scale) {
  const int nd = x->ndim;
  if (dim < 0) dim += nd;
  if (dim < 0 || dim >= nd) fail("sum dim %lld out of range for %d-D tensor", (long long)dim, nd);
  check_dtype("sum_dim", kNotBool, x->dtype);
  TensorP c = contiguous(x);
  int64_t outer = 1, inner = 1;
  for (int i = 0; i < dim; ++i) outer *= c->shape[i];
  for (int i = (int)dim + 1; i < nd; ++i) inner *= c->shape[i];
  std::vector<int64_t> od;
  for (int i = 0; i < nd; ++i) {
    if (i == dim) { if (keepdim) od.push_back(1); }
    else od.push_back(c->shape[i]);
  }
  if (od.empty()) od = {1};
  TensorP out = alloc_out(c->dtype, od);
  LAUNCH k::sum_dim(c->dtype, c->data(), out->data(), outer, c->shape[dim], inner, scale, rt().stream());
  return out;
}

TensorP mean_all(const TensorP& x) {
  if (x->ndim == 0) fail("mean_all requires at least 1D tensor");
  check_dtype("mean_all", kFloatOnly, x->dtype);
  TensorP c = contiguous(x);
  TensorP out = alloc_out(c->dtype, {1});
  BufferP ws = scratch(k::reduce_all_ws_bytes());
  int64_t n = c->numel();
  LAUNCH k::reduce_all(0, c->dtype, c->data(), nullptr, n, n ? 1.f / (float)n : NAN, out->data(), ws->ptr, rt().stream());
  return out;
}

TensorP mse_loss(const TensorP& a, const TensorP& b) {
  if (a->dims() != b->dims()) fail("mse_loss: shape mismatch %s vs %s", shape_str(a->dims()).c_str(),
                                   shape_str(b->dims()).c_str());
  if (a->dtype != b->dtype) fail("mse_loss: dtype mismatch");
  check_dtype("mse_loss", kFloatOnly, a->dtype);
  TensorP ac = contiguous(a), bc = contiguous(b);
  TensorP out = alloc_out(a->dtype, {1});
  BufferP ws = scratch(k::reduce_all_ws_bytes());
  int64_t n = ac->numel();
  LAUNCH k::reduce_all(1, a->dtype, ac->data(), bc->data(), n, n ? 1.f / (float)n : NAN, out->data(), ws->ptr, rt().stream());
  return out;
}

TensorP mse_loss_backward(const TensorP& g, const TensorP& a, const TensorP& b) {
  if (a->dims() != b->dims()) fail("mse_loss_backward: shape mismatch");
  if (g->numel() != 1) fail("mse_loss_backward: grad_output must have one element");
  if (a->dtype != b->dtype || g->dtype != a->dtype) fail("mse_loss_backward: dtype mismatch");
  check_dtype("mse_loss_backward", kFloatOnly, a->dtype);
  TensorP ac = contiguous(a), bc = contiguous(b);
  TensorP out = alloc_out(a->dtype, a->dims());
  LAUNCH k::mse_backward(a->dtype, ac->data(), bc->data(), g->data(), out->data(), ac->numel(), rt().stream());
  return out;
}

std::pair<TensorP, TensorP> mse_loss_grad(const TensorP& a, const TensorP& b) {
  if (a->dims() != b->dims()) fail("mse_loss_grad: shape mismatch %s vs %s", shape_str(a->dims()).c_str(),
                                   shape_str(b->dims()).c_str());
  if (a->dtype != b->dtype) fail("mse_loss_grad: dtype mismatch");
  check_dtype("mse_loss_grad", kFloatOnly, a->dtype);
  const int64_t n = a->numel();
  if (!k::mse_fused_ok(n)) {
    TensorP one = full(a->dtype, {1}, 1.f);
    return {mse_loss(a, b), mse_loss_backward(one, a, b)};
  }
  TensorP ac = contiguous(a), bc = contiguous(b);
  TensorP loss = alloc_out(a->dtype, {1});
  TensorP grad = alloc_out(a->dtype, a->dims());
  LAUNCH k::mse_loss_grad(a->dtype, ac->data(), bc->data(), loss->data(), grad->data(), n, rt().stream());
  return {loss, grad};
}

TensorP sgd_matmul_(const TensorP& w, const TensorP& a, const TensorP& b, bool ta, bool tb, float alpha,
                    const TensorP& bias) {
  if (w->ndim != 2) fail("sgd_matmul_: the parameter must be 2-D");
  Epilogue e;
  e.alpha = alpha;
  e.residual = w;
  e.a_rowsum_acc = bias;
  return matmul(a, b, ta, tb, &e, w);
}

TensorP linear_backward_sgd_(const TensorP& w, const TensorP& b, const TensorP& g, const TensorP& a,
                             const TensorP& mask, float alpha) {
  if (w->ndim != 2 || g->ndim != 2 || a->ndim != 2)
    fail("linear_backward_sgd_: w, g and a must be 2-D");
  const int64_t R = g->shape[0], O = w->shape[0], N = w->shape[1];
  if (g->shape[1] != O || a->shape[0] != R || a->shape[1] != N)
    fail("linear_backward_sgd_: g %s and a %s do not fit w %s", shape_str(g->dims()).c_str(),
         shape_str(a->dims()).c_str(), shape_str(w->dims()).c_str());
  if (b->numel() != O) fail("linear_backward_sgd_: bias must have %lld elements", (long long)O);
  if (mask && mask->dims() != a->dims()) fail("linear_backward_sgd_: the mask must have a's shape");
  const bool f32 = w->dtype == DType::F32 && b->dtype == DType::F32 && g->dtype == DType::F32 &&
                   a->dtype == DType::F32;
  if (O == 1 && f32 && w->is_contiguous() && b->is_contiguous() && a->strides[1] == 1 &&
      (!mask || mask.get() == a.get())) {
    TensorP gin = mask ? alloc_out(DType::F32, {R, N}) : nullptr;
    k::Lin1Bwd p{a->data(), a->strides[0], g->data(), g->strides[0], w->data(), b->data(),
                 gin ? gin->data() : nullptr, R, N, alpha};
    LAUNCH k::linear1_backward_sgd(DType::F32, p, rt().stream());
    return gin ? gin : w;
  }
  TensorP gin;
  if (mask) {
    Epilogue e;
    e.mask = mask;
    gin = matmul(g, w, false, false, &e);
  }
  sgd_matmul_(w, g, a, true, false, alpha, b);
  return mask ? gin : w;
}

TensorP mlp2_sgd_step_(const TensorP& x, const TensorP& y, const TensorP& w1, const TensorP& b1, const TensorP& w2,
                       const TensorP& b2, float alpha) {
  const char* name = "mlp2_sgd_step_";
  if (x->ndim != 2 || w1->ndim != 2 || w2->ndim != 2 || y->ndim != 2) fail("%s: x, y, w1 and w2 must be 2-D", name);
  const int64_t R = x->shape[0], N0 = x->shape[1], N1 = w1->shape[0], N2 = w2->shape[0];
  if (w1->shape[1] != N0 || w2->shape[1] != N1 || b1->numel() != N1 || b2->numel() != N2 ||
      y->dims() != std::vector<int64_t>{R, N2})
    fail("%s: x %s, w1 %s, b1 %s, w2 %s, b2 %s and y %s do not form Linear -> ReLU -> Linear", name,
         shape_str(x->dims()).c_str(), shape_str(w1->dims()).c_str(), shape_str(b1->dims()).c_str(),
         shape_str(w2->dims()).c_str(), shape_str(b2->dims()).c_str(), shape_str(y->dims()).c_str());
  const bool f32 = x->dtype == DType::F32 && y->dtype == DType::F32 && w1->dtype == DType::F32 &&
                   b1->dtype == DType::F32 && w2->dtype == DType::F32 && b2->dtype == DType::F32;
  const bool contig = x->is_contiguous() && y->is_contiguous() && w1->is_contiguous() && b1->is_contiguous() &&
                      w2->is_contiguous() && b2->is_contiguous();
  const bool al16 = (((uintptr_t)x->data() | (uintptr_t)w1->data() | (uintptr_t)w2->data()) & 15) == 0;
  if (f32 && contig && al16 && k::mlp2_step_ok(R, N0, N1, N2)) {
    TensorP loss = alloc_out(DType::F32, {1});
    k::Mlp2Step a{(const float*)x->data(), (const float*)y->data(), (float*)w1->data(), (float*)b1->data(),
                  (float*)w2->data(), (float*)b2->data(), (float*)loss->data(),
                  (int)R, (int)N0, (int)N1, (int)N2, alpha};
    LAUNCH k::mlp2_step(a, rt().stream());
    return loss;
  }
  Epilogue e;
  e.bias = b1;
  e.act = k::kActRelu;
  TensorP h = matmul(x, w1, false, true, &e);
  auto r = linear_mse_backward_sgd_(h, w2, b2, y, alpha, true);
  linear_backward_sgd_(w1, b1, r.second, x, nullptr, alpha);
  return r.first;
}

std::pair<TensorP, TensorP> linear_mse_backward_sgd_(const TensorP& h, const TensorP& w, const TensorP& b,
                                                     const TensorP& y, float alpha, bool grad_in) {
  if (h->ndim != 2 || w->ndim != 2) fail("linear_mse_backward_sgd_: h and w must be 2-D");
  const int64_t R = h->shape[0], N = h->shape[1], O = w->shape[0];
  if (w->shape[1] != N) fail("linear_mse_backward_sgd_: w %s does not fit h %s", shape_str(w->dims()).c_str(),
                             shape_str(h->dims()).c_str());
  if (b->numel() != O) fail("linear_mse_backward_sgd_: bias must have %lld elements", (long long)O);
  if (y->dims() != std::vector<int64_t>{R, O})
    fail("linear_mse_backward_sgd_: y must be [%lld, %lld]", (long long)R, (long long)O);
  const bool f32 = h->dtype == DType::F32 && w->dtype == DType::F32 && b->dtype == DType::F32 &&
                   y->dtype == DType::F32;
  if (O == 1 && R > 0 && f32 && h->strides[1] == 1 && w->is_contiguous() && b->is_contiguous() &&
      y->is_contiguous()) {
    TensorP z = alloc_out(DType::F32, {R, 1}), dz = alloc_out(DType::F32, {R, 1});
    TensorP loss = alloc_out(DType::F32, {1});
    TensorP gin = grad_in ? alloc_out(DType::F32, {R, N}) : nullptr;
    const float n = (float)R;
    k::Lin1Fwd f{h->data(), h->strides[0], w->data(), b->data(), y->data(), z->data(), dz->data(), R, N, 2.f / n};
    LAUNCH k::linear1_forward_mse(DType::F32, f, rt().stream());
    k::Lin1Bwd p{h->data(), h->strides[0], dz->data(), 1, w->data(), b->data(), gin ? gin->data() : nullptr,
                 R, N, alpha, z->data(), y->data(), loss->data(), 1.f / n};
    LAUNCH k::linear1_backward_sgd(DType::F32, p, rt().stream());
    return {loss, gin ? gin : w};
  }
  Epilogue e;
  e.bias = b;
  TensorP out = matmul(h, w, false, true, &e);
  auto lg = mse_loss_grad(out, y);
  TensorP gi = linear_backward_sgd_(w, b, lg.second, h, grad_in ? h : nullptr, alpha);
  return {lg.first, gi};
}

std::tuple<TensorP, TensorP, TensorP> linear_relu_mse_backward_sgd_(const TensorP& a, const TensorP& wh,
                                                                    const TensorP& bh, const TensorP& w,
                                                                    const TensorP& b, const TensorP& y, float alpha,
                                                                    bool grad_in) {
  const char* name = "linear_relu_mse_backward_sgd_";
  if (a->ndim != 2 || wh->ndim != 2) fail("%s: a and wh must be 2-D", name);
  const int64_t R = a->shape[0], K = a->shape[1], N = wh->shape[0];
  if (wh->shape[1] != K || bh->numel() != N)
    fail("%s: wh %s and bh %s do not fit a %s", name, shape_str(wh->dims()).c_str(), shape_str(bh->dims()).c_str(),
         shape_str(a->dims()).c_str());
  auto layered = [&]() {
    Epilogue e;
    e.bias = bh;
    e.act = k::kActRelu;
    TensorP h = matmul(a, wh, false, true, &e);
    auto r = linear_mse_backward_sgd_(h, w, b, y, alpha, grad_in);
    return std::make_tuple(r.first, r.second, h);
  };
  const bool f32 = a->dtype == DType::F32 && wh->dtype == DType::F32 && bh->dtype == DType::F32 &&
                   w->dtype == DType::F32 && b->dtype == DType::F32 && y->dtype == DType::F32;
  if (meta_mode() || !f32 || w->ndim != 2 || w->shape[0] != 1 || w->shape[1] != N || b->numel() != 1 ||
      y->dims() != std::vector<int64_t>{R, 1} || N % 4 != 0 || !a->is_contiguous() || !wh->is_contiguous() ||
      !bh->is_contiguous() || !w->is_contiguous() || !b->is_contiguous() || !y->is_contiguous())
    return layered();
  // h's GEMM with its split-K partial sums left for the output layer's
  // forward, which reduces them (bias, ReLU) while it forms z
  k::Gemm g;
  g.dt = g.b_dt = DType::F32;
  g.M = R; g.N = N; g.K = K; g.batch = 1;
  g.A = a->data(); g.a_sm = K; g.a_sk = 1; g.a_sb = R * K;
  g.B = wh->data(); g.b_sk = 1; g.b_sn = K; g.b_sb = N * K;
  g.C = nullptr; g.c_sm = N; g.c_sb = R * N;
  g.no_reduce = true;
  const int splits = k::gemm_splits(g);
  if (splits < 2 || splits > 8) return layered();
  BufferP ws = scratch(k::gemm_workspace_bytes(g));
  LAUNCH k::gemm(g, ws->ptr, rt().stream());
  TensorP h = alloc_out(DType::F32, {R, N});
  TensorP z = alloc_out(DType::F32, {R, 1}), dz = alloc_out(DType::F32, {R, 1});
  TensorP loss = alloc_out(DType::F32, {1});
  TensorP gin = grad_in ? alloc_out(DType::F32, {R, N}) : nullptr;
  const float n = (float)R;
  k::Lin1FwdParts f{(const float*)ws->ptr, splits, R * N, (const float*)bh->data(), (float*)h->data(),
                    (const float*)w->data(), (const float*)b->data(), (const float*)y->data(), (float*)z->data(),
                    (float*)dz->data(), R, N, 2.f / n};
  LAUNCH k::linear1_forward_mse_parts(f, rt().stream());
  k::Lin1Bwd p{h->data(), N, dz->data(), 1, w->data(), b->data(), gin ? gin->data() : nullptr,
               R, N, alpha, z->data(), y->data(), loss->data(), 1.f / n};
  LAUNCH k::linear1_backward_sgd(DType::F32, p, rt().stream());
  return std::make_tuple(loss, gin ? gin : w, h);
}

TensorP sgd_sum_rows_(const TensorP& bias, const TensorP& g, float alpha) {
  check_dtype("sgd_sum_rows_", kFloatOnly, g->dtype);
  if (g->ndim != 2 || bias->dtype != g->dtype || bias->numel() != g->shape[1] || !bias->is_contiguous())
    fail("sgd_sum_rows_: bias must be a contiguous [%lld] tensor of the gradient's dtype",
         (long long)(g->ndim == 2 ? g->shape[1] : -1));
  TensorP gc = contiguous(g);
  LAUNCH k::sum_rows_axpy(g->dtype, gc->data(), bias->data(), gc->shape[0], gc->shape[1], alpha, rt().stream());
  return bias;
}

// ── indexing ───────────────────────────────────────────────────────────────
TensorP embedding(const TensorP& w, const TensorP& idx) {
  if (w->ndim != 2) fail("embedding weights must be 2D [vocab_size, embed_dim]");
  if (idx->ndim < 1) fail("embedding indices must have at least 1 dimension");
  if (idx->dtype != DType::I32 && idx->dtype != DType::I64)
    fail("embedding indices must be Int32, got %s", dtype_name(idx->dtype));
  TensorP wc = contiguous(w), ic = contiguous(idx);
  std::vector<int64_t> od = idx->dims();
  od.push_back(w->shape[1]);
  TensorP out = alloc_out(w->dtype, od);
  LAUNCH k::embedding(w->dtype, wc->data(), w->shape[0], w->shape[1], ic->dtype, ic->data(), ic->numel(), out->data(),
               rt().stream());
  return out;
}

bool embedding_add_fusable(const TensorP& w1, const TensorP& i1, const TensorP& w2, const TensorP& i2) {
  return w1->ndim == 2 && w2->ndim == 2 && w1->dtype == w2->dtype && dtype_is_float(w1->dtype) &&
         w1->dtype != DType::F64 && w1->shape[1] == w2->shape[1] && k::embedding_add_ok(w1->shape[1]) &&
         i1->dtype == i2->dtype && (i1->dtype == DType::I32 || i1->dtype == DType::I64) && i1->dims() == i2->dims() &&
         w1->is_contiguous() && w2->is_contiguous();
}

TensorP embedding_add(const TensorP& w1, const TensorP& i1, const TensorP& w2, const TensorP& i2, PostLn* ln) {
  if (!embedding_add_fusable(w1, i1, w2, i2)) fail("embedding_add: operands do not fit the fused kernel");
  TensorP a = contiguous(i1), c = contiguous(i2);
  std::vector<int64_t> od = i1->dims();
  od.push_back(w1->shape[1]);
  TensorP x = alloc_out(w1->dtype, od);
  const int64_t rows = a->numel(), cols = w1->shape[1];
  TensorP gc, bc;
  if (ln) {
    if (!(ln->gamma->ndim == 1 && ln->gamma->shape[0] == cols && ln->beta->ndim == 1 && ln->beta->shape[0] == cols &&
          ln->gamma->dtype == w1->dtype && ln->beta->dtype == w1->dtype))
      fail("embedding_add: layer_norm gamma/beta must be [%lld] of the table dtype", (long long)cols);
    gc = contiguous(ln->gamma);
    bc = contiguous(ln->beta);
    if (ln->want_pk && (w1->dtype != DType::F32 || cols % 16 != 0 || od.size() != 2))
      fail("embedding_add: packed layer_norm rows need fp32 [rows, cols] with cols %% 16 == 0");
    ln->y = ln->want_y ? alloc_out(w1->dtype, od) : nullptr;
    ln->ypk = ln->want_pk ? alloc_out(DType::BF16, {(rows + 31) / 32, cols / 16, 2, 64, 8}) : nullptr;
  }
  LAUNCH k::embedding_add(w1->dtype, w1->data(), a->dtype, a->data(), w1->shape[0], w2->data(), c->dtype, c->data(),
                          w2->shape[0], x->data(), ln ? gc->data() : nullptr, ln ? bc->data() : nullptr,
                          ln && ln->y ? ln->y->data() : nullptr, ln && ln->ypk ? ln->ypk->data() : nullptr, rows,
                          cols, ln ? ln->eps : 1e-5f, rt().stream());
  return x;
}

TensorP index_select(const TensorP& x, int dim, const TensorP& idx) {
  check_dtype("index_select", kNotBool, x->dtype);
  if (idx->ndim != 1) fail("index_select index must be 1D");
  if (idx->dtype != DType::I32 && idx->dtype != DType::I64) fail("index_select indices must be Int32");
  if (dim < 0 || dim >= x->ndim) fail("index_select dim %d out of range", dim);
  TensorP c = contiguous(x), ic = contiguous(idx);
  int64_t outer = 1, inner = 1;
  for (int i = 0; i < dim; ++i) outer *= c->shape[i];
  for (int i = dim + 1; i < c->ndim; ++i) inner *= c->shape[i];
  auto od = c->dims();
  od[dim] = idx->shape[0];
  TensorP out = alloc_out(c->dtype, od);
  LAUNCH k::index_select(c->dtype, c->data(), outer, c->shape[dim], inner, ic->dtype, ic->data(), idx->shape[0],
                  out->data(), rt().stream());
  return out;
}

TensorP gather(const TensorP& x, int dim, const TensorP& idx) {
  check_dtype("gather", kNotBool, x->dtype);
  if (idx->dtype != DType::I32 && idx->dtype != DType::I64) fail("gather indices must be Int32");
  if (idx->ndim != x->ndim) fail("gather index must have the same ndim as the input");
  if (dim < 0 || dim >= x->ndim) fail("gather dim %d out of range", dim);
  for (int i = 0; i < x->ndim; ++i)
    if (i != dim && idx->shape[i] != x->shape[i])
      fail("gather dim=%d: index dim %d (%lld) must match input (%lld)", dim, i, (long long)idx->shape[i],
           (long long)x->shape[i]);
  TensorP c = contiguous(x), ic = contiguous(idx);
  int64_t outer = 1, inner = 1;
  for (int i = 0; i < dim; ++i) outer *= c->shape[i];
  for (int i = dim + 1; i < c->ndim; ++i) inner *= c->shape[i];
  TensorP out = alloc_out(c->dtype, idx->dims());
  LAUNCH k::gather(c->dtype, c->data(), outer, c->shape[dim], inner, ic->dtype, ic->data(), idx->shape[dim], out->data(),
            rt().stream());
  return out;
}

TensorP concat(const TensorP& a, const TensorP& b, int dim) {
  if (a->dtype != b->dtype) fail("concat dtype mismatch: %s vs %s", dtype_name(a->dtype), dtype_name(b->dtype));
  if (a->ndim != b->ndim) fail("concat ndim mismatch: %s vs %s", shape_str(a->dims()).c_str(), shape_str(b->dims()).c_str());
  if (dim < 0 || dim >= a->ndim) fail("concat dim %d >= ndim %d", dim, a->ndim);
  for (int i = 0; i < a->ndim; ++i)
    if (i != dim && a->shape[i] != b->shape[i])
      fail("concat shape mismatch on dim %d: %lld vs %lld", i, (long long)a->shape[i], (long long)b->shape[i]);
  auto od = a->dims();
  od[dim] += b->shape[dim];
  TensorP out = alloc_out(a->dtype, od);
  // Each half is a strided copy into a slice of the output.
  TensorP oa = slice(out, dim, 0, a->shape[dim]);
  auto ad = a->dims();
  k::ND so_a = nd_for(*oa, ad);
  // Copy kernels write contiguously; write each half as "out slice = in" by
  // iterating in the output slice's index space through a temporary when the
  // slice is not contiguous (dim > 0).
  if (dim == 0) {
    LAUNCH k::unary(k::kCopy, a->dtype, a->dtype, a->data(), nd_for(*a, ad), oa->data(), nd_shape(ad), 0, 0, rt().stream());
    TensorP ob = slice(out, dim, a->shape[dim], od[dim]);
    auto bd = b->dims();
    LAUNCH k::unary(k::kCopy, b->dtype, b->dtype, b->data(), nd_for(*b, bd), ob->data(), nd_shape(bd), 0, 0, rt().stream());
    (void)so_a;
    return out;
  }
  // General dim: build the output as where(select) over a broadcast index is
  // wasteful; instead move `dim` to the front, concat there, and move back.
  TensorP at = contiguous(transpose_dims(a, 0, dim));
  TensorP bt = contiguous(transpose_dims(b, 0, dim));
  TensorP ct = concat(at, bt, 0);
  return contiguous(transpose_dims(ct, 0, dim));
}

// ── GEMM ───────────────────────────────────────────────────────────────────
// Collapse the (already broadcast) batch dims of an operand into one stride.
static bool batch_stride(const Tensor& t, const std::vector<int64_t>& bdims, int64_t* stride) {
  // strides of t's batch dims aligned to bdims (0 = broadcast)
  const int nb = (int)bdims.size();
  const int tb = t.ndim - 2;
  std::vector<int64_t> st(nb, 0);
  for (int i = 0; i < nb; ++i) {
    int ti = i - (nb - tb);
    if (ti >= 0 && t.shape[ti] == bdims[i] && bdims[i] != 1) st[i] = t.strides[ti];
  }
  // collapsible if st[i] == st[i+1] * bdims[i+1] for non-unit dims
  int64_t s = -1, expect = 0;
  for (int i = nb - 1; i >= 0; --i) {
    if (bdims[i] == 1) continue;
    if (s < 0) { s = st[i]; expect = st[i] * bdims[i]; continue; }
    if (st[i] != expect) return false;
    expect *= bdims[i];
  }
  *stride = s < 0 ? 0 : s;
  return true;
}

// Epilogue operands of a GEMM (bias, residual, mask, layer-norm prologue);
// `keep` holds the tensors the launch reads.
struct EpiKeep {
  TensorP res, mask, bias, ln_g, ln_b;
};

static void set_epilogue(k::Gemm& g, const Epilogue* epi, const std::vector<int64_t>& od,
                         const std::vector<int64_t>& bdims, EpiKeep* keep) {
  if (!epi) return;
  const int64_t M = g.M, N = g.N;
  g.alpha = epi->alpha;
  g.act = epi->act;
  if (epi->bias) {
    if (epi->bias->dtype != g.dt || epi->bias->numel() != N) fail("matmul epilogue: bias must be [%lld]", (long long)N);
    keep->bias = contiguous(epi->bias);
    g.bias = keep->bias->data();
  }
  if (epi->ln_gamma) {
    if (!epi->ln_beta || epi->ln_gamma->dtype != g.dt || epi->ln_beta->dtype != g.dt ||
        epi->ln_gamma->numel() != g.K || epi->ln_beta->numel() != g.K)
      fail("matmul: layer-norm gamma and beta must be [%lld] of the operand dtype", (long long)g.K);
    keep->ln_g = contiguous(epi->ln_gamma);
    keep->ln_b = contiguous(epi->ln_beta);
    g.ln_gamma = keep->ln_g->data();
    g.ln_beta = keep->ln_b->data();
    g.ln_eps = epi->ln_eps;
  }
  auto side = [&](const TensorP& t, const void** ptr, int64_t* sm, int64_t* sb, TensorP* kp) {
    if (t->dtype != g.dt) fail("matmul epilogue: operand dtype mismatch");
    if (t->dims() != od) {
      // broadcast residual: expand through strides (must collapse)
      *kp = alloc_out(g.dt, od);
      LAUNCH k::unary(k::kCopy, t->dtype, t->dtype, t->data(), nd_for(*t, od), (*kp)->data(), nd_shape(od), 0, 0,
               rt().stream());
    } else {
      *kp = t;
    }
    const Tensor& r = **kp;
    int64_t rsb;
    if (r.strides[r.ndim - 1] != 1 && N > 1) { *kp = contiguous(*kp); }
    const Tensor& r2 = **kp;
    if (!batch_stride(r2, bdims, &rsb)) { *kp = contiguous(*kp); batch_stride(**kp, bdims, &rsb); }
    *ptr = (*kp)->data();
    *sm = (*kp)->strides[(*kp)->ndim - 2];
    if (M == 1) *sm = N;
    *sb = rsb;
  };
  if (epi->residual) side(epi->residual, &g.residual, &g.r_sm, &g.r_sb, &keep->res);
  if (epi->mask) side(epi->mask, &g.mask, &g.k_sm, &g.k_sb, &keep->mask);
}

TensorP matmul(const TensorP& a_in, const TensorP& b_in, bool ta, bool tb, const Epilogue* epi, const TensorP& into,
               PostLn* post_ln, const NoAlloc* no_alloc) {
  if (no_alloc) {
    // Everything below must then run without a device allocation.
    if (meta_mode()) fail("matmul: the allocation-free form runs eagerly only");
    if (!into) fail("matmul: the allocation-free form writes into a caller-provided output");
    if (post_ln) fail("matmul: the allocation-free form takes no layer_norm");
    if (epi && (epi->ln_gamma || epi->residual || epi->mask || epi->a_rowsum_acc))
      fail("matmul: the allocation-free form takes a bias and an activation only");
    if (epi && epi->bias && !epi->bias->is_contiguous())
      fail("matmul: the allocation-free form needs a contiguous bias (a copy would allocate)");
  }
  TensorP a = ta ? transpose_dims(a_in, a_in->ndim - 2, a_in->ndim - 1) : a_in;
  TensorP b = tb ? transpose_dims(b_in, b_in->ndim - 2, b_in->ndim - 1) : b_in;
  if (a_in->ndim < 2 || b_in->ndim < 2) fail("matmul requires at least 2D tensors, got %s and %s",
                                             shape_str(a_in->dims()).c_str(), shape_str(b_in->dims()).c_str());
  check_dtype("matmul", kFloatOnly, a->dtype);
  if (a->dtype != b->dtype) fail("Dtype mismatch: %s vs %s", dtype_name(a->dtype), dtype_name(b->dtype));
  const int64_t M = a->shape[a->ndim - 2], K = a->shape[a->ndim - 1];
  const int64_t K2 = b->shape[b->ndim - 2], N = b->shape[b->ndim - 1];
  if (K != K2)
    fail("matmul inner dimensions mismatch: A[...,%lld,%lld] * B[...,%lld,%lld]", (long long)M, (long long)K,
         (long long)K2, (long long)N);
  std::vector<int64_t> ab(a->shape, a->shape + a->ndim - 2), bb(b->shape, b->shape + b->ndim - 2);
  std::vector<int64_t> bdims = broadcast_shapes(ab.empty() ? std::vector<int64_t>{1} : ab,
                                                bb.empty() ? std::vector<int64_t>{1} : bb);
  std::vector<int64_t> od = bdims;
  if (ab.empty() && bb.empty()) od.clear();
  od.push_back(M);
  od.push_back(N);
  int64_t batch = 1;
  for (auto d : bdims) batch *= d;

  int64_t a_sb, b_sb;
  if (no_alloc && (!batch_stride(*a, bdims, &a_sb) || !batch_stride(*b, bdims, &b_sb)))
    fail("matmul: an operand's batch layout needs a copy, which the allocation-free form cannot make");
  if (!batch_stride(*a, bdims, &a_sb)) {
    // expand to the broadcast batch shape, contiguous
    std::vector<int64_t> full = bdims;
    full.push_back(M); full.push_back(K);
    TensorP ex = alloc_out(a->dtype, full);
    LAUNCH k::unary(k::kCopy, a->dtype, a->dtype, a->data(), nd_for(*a, full), ex->data(), nd_shape(full), 0, 0, rt().stream());
    a = ex;
    batch_stride(*a, bdims, &a_sb);
  }
  if (!batch_stride(*b, bdims, &b_sb)) {
    std::vector<int64_t> full = bdims;
    full.push_back(K); full.push_back(N);
    TensorP ex = alloc_out(b->dtype, full);
    LAUNCH k::unary(k::kCopy, b->dtype, b->dtype, b->data(), nd_for(*b, full), ex->data(), nd_shape(full), 0, 0, rt().stream());
    b = ex;
    batch_stride(*b, bdims, &b_sb);
  }
  TensorP out;
  if (into) {
    // caller-provided output (may also be the residual: each output element
    // is read and written by the same thread of the epilogue)
    if (into->dtype != a->dtype || into->dims() != od || !into->is_contiguous())
      fail("matmul: output must be a contiguous %s tensor of shape %s", dtype_name(a->dtype), shape_str(od).c_str());
    out = into;
  } else {
    out = alloc_out(a->dtype, od);
  }

  k::Gemm g;
  g.dt = a->dtype;
  g.b_dt = b->dtype;
  g.M = M; g.N = N; g.K = K; g.batch = batch;
  g.A = a->data(); g.a_sm = a->strides[a->ndim - 2]; g.a_sk = a->strides[a->ndim - 1]; g.a_sb = a_sb;
  g.B = b->data(); g.b_sk = b->strides[b->ndim - 2]; g.b_sn = b->strides[b->ndim - 1]; g.b_sb = b_sb;
  // Unit extents: pick the stride that makes the operand look contiguous.
  if (M == 1) g.a_sm = g.a_sk == 1 ? K : 1;
  if (K == 1) { if (g.a_sm != 1) g.a_sk = 1; if (g.b_sn != 1) g.b_sk = 1; }
  if (N == 1) g.b_sn = g.b_sk == 1 ? K : 1;
  g.C = out->data(); g.c_sm = N; g.c_sb = M * N;
  if (epi && epi->ln_gamma) {
    bool ok = !ta && a_in->ndim == 2 && b_in->ndim == 2 && epi->ln_beta && epi->ln_gamma->dtype == g.dt &&
              epi->ln_beta->dtype == g.dt && epi->ln_gamma->numel() == K && epi->ln_beta->numel() == K;
    if (ok) {
      k::Gemm probe = g;
      probe.ln_gamma = epi->ln_gamma->data();
      probe.ln_beta = epi->ln_beta->data();
      ok = meta_mode() ? k::gemm_is_skinny(probe) : (epi->ln_gamma->is_contiguous() && epi->ln_beta->is_contiguous() &&
                                                     k::gemm_skinny_ln_ok(probe));
    }
    if (!ok) {
      Epilogue plain = *epi;
      plain.ln_gamma = plain.ln_beta = nullptr;
      return matmul(layer_norm(a_in, epi->ln_gamma, epi->ln_beta, epi->ln_eps), b_in, ta, tb, &plain, into, post_ln);
    }
  }
  EpiKeep keep;
  set_epilogue(g, epi, od, bdims, &keep);
  bool rowsum_fused = false;
  if (epi && epi->a_rowsum_acc) {
    const TensorP& acc = epi->a_rowsum_acc;
    if (acc->dtype != DType::F32 || g.dt != DType::F32 || a_in->ndim != 2 || b_in->ndim != 2 ||
        acc->numel() != M || !acc->is_contiguous())
      fail("matmul: the row-sum accumulator must be a contiguous fp32 [%lld] tensor beside a 2-D fp32 product",
           (long long)M);
    if (!meta_mode()) {
      k::Gemm probe = g;
      probe.a_rowsum_acc = acc->data();
      rowsum_fused = k::gemm_a_rowsum_fused(probe);
      if (rowsum_fused) g = probe;
    }
  }
  TensorP pl_g, pl_b;
  bool pln_fused = false;
  if (post_ln) {
    if (!post_ln->gamma || !post_ln->beta || post_ln->gamma->dtype != g.dt || post_ln->beta->dtype != g.dt ||
        post_ln->gamma->numel() != N || post_ln->beta->numel() != N)
      fail("matmul: layer_norm gamma and beta must be [%lld] of the output dtype", (long long)N);
    pl_g = contiguous(post_ln->gamma);
    pl_b = contiguous(post_ln->beta);
    if (!meta_mode()) {
      TensorP y = alloc_out(g.dt, od);
      k::Gemm probe = g;
      probe.pln_gamma = pl_g->data();
      probe.pln_beta = pl_b->data();
      probe.pln_y = y->data();
      probe.pln_eps = post_ln->eps;
      pln_fused = k::gemm_post_ln_fused(probe);
      if (pln_fused) {
        g = probe;
        post_ln->y = y;
      }
    }
  }
  // the allocation-free form: plans whose workspace would not fit the
  // static scratch (the outer-product plan's packed operands) are skipped
  if (no_alloc) g.max_ws = no_alloc->cap;
  size_t wsb = meta_mode() ? 0 : k::gemm_workspace_bytes(g);
  if (no_alloc) {
    if (wsb > no_alloc->cap)
      fail("matmul: this %lld x %lld x %lld product needs %zu bytes of workspace (split-K partial sums or "
           "packed operands), more than the %zu bytes the allocation-free form holds",
           (long long)M, (long long)N, (long long)K, wsb, no_alloc->cap);
    LAUNCH k::gemm(g, wsb ? no_alloc->ws : nullptr, rt().stream());
    return out;
  }
  BufferP ws;
  if (wsb) ws = scratch(wsb);
  LAUNCH k::gemm(g, ws ? ws->ptr : nullptr, rt().stream());
  if (post_ln && !pln_fused) post_ln->y = layer_norm(out, pl_g, pl_b, post_ln->eps);
  if (epi && epi->a_rowsum_acc && !rowsum_fused) {
    // the row sums of op(a) on their own: op(a) = a_in^T with a_in a
    // contiguous [K, M] gradient is the column-sum kernel of sgd_sum_rows_
    const TensorP& acc = epi->a_rowsum_acc;
    if (ta && a_in->is_contiguous()) {
      LAUNCH k::sum_rows_axpy(DType::F32, a_in->data(), acc->data(), K, M, epi->alpha, rt().stream());
    } else {
      axpy_inplace(acc, sum_dim(a, 1, false, 1.f), epi->alpha);
    }
  }
  return out;
}

// The SGD step w += alpha g^T a with b += alpha sum(g, 0) as the Gemm that
// sgd_matmul_(w, g, a, true, false, alpha, b) hands to k::gemm (A = g^T read
// in place, the residual and output w, the bias as A's row-sum
// accumulator); false when an operand is not plain contiguous fp32.
static bool sgd_update_gemm(const TensorP& w, const TensorP& b, const TensorP& g, const TensorP& a, float alpha,
                            k::Gemm& G, EpiKeep& keep) {
  for (const TensorP* t : {&w, &b, &g, &a})
    if ((*t)->dtype != DType::F32 || !(*t)->is_contiguous()) return false;
  const int64_t R = g->shape[0], O = w->shape[0], N = w->shape[1];
  if (R < 2 || O < 2 || N < 2) return false;
  G = k::Gemm{};
  G.dt = G.b_dt = DType::F32;
  G.M = O; G.N = N; G.K = R; G.batch = 1;
  G.A = g->data(); G.a_sm = g->strides[1]; G.a_sk = g->strides[0]; G.a_sb = 0;
  G.B = a->data(); G.b_sk = a->strides[0]; G.b_sn = a->strides[1]; G.b_sb = 0;
  G.C = w->data(); G.c_sm = N; G.c_sb = O * N;
  Epilogue e;
  e.alpha = alpha;
  e.residual = w;
  set_epilogue(G, &e, {O, N}, {1}, &keep);
  G.a_rowsum_acc = b->data();
  return true;
}

TensorP linear_backward_sgd_pair_(const TensorP& w1, const TensorP& b1, const TensorP& g, const TensorP& h,
                                  const TensorP& w0, const TensorP& b0, const TensorP& x, float alpha) {
  const char* name = "linear_backward_sgd_pair_";
  if (w1->ndim != 2 || g->ndim != 2 || h->ndim != 2 || w0->ndim != 2 || x->ndim != 2)
    fail("%s: w1, g, h, w0 and x must be 2-D", name);
  const int64_t R = g->shape[0], O1 = w1->shape[0], N1 = w1->shape[1], N0 = w0->shape[1];
  if (g->shape[1] != O1 || h->dims() != std::vector<int64_t>{R, N1} || w0->shape[0] != N1 ||
      x->dims() != std::vector<int64_t>{R, N0} || b1->numel() != O1 || b0->numel() != N1)
    fail("%s: g %s, h %s, x %s, w1 %s, b1 %s, w0 %s and b0 %s do not form two stacked Linear layers", name,
         shape_str(g->dims()).c_str(), shape_str(h->dims()).c_str(), shape_str(x->dims()).c_str(),
         shape_str(w1->dims()).c_str(), shape_str(b1->dims()).c_str(), shape_str(w0->dims()).c_str(),
         shape_str(b0->dims()).c_str());
  // the lower layer's output gradient through its ReLU, from w1 before its step
  Epilogue e;
  e.mask = h;
  TensorP g0 = matmul(g, w1, false, false, &e);
  k::Gemm G1, G0;
  EpiKeep k1, k0;
  if (!meta_mode() && sgd_update_gemm(w1, b1, g, h, alpha, G1, k1) && sgd_update_gemm(w0, b0, g0, x, alpha, G0, k0) &&
      k::gemm_outer_pair_ok(G1, G0)) {
    BufferP ws1 = scratch(k::gemm_workspace_bytes(G1)), ws0 = scratch(k::gemm_workspace_bytes(G0));
    k::gemm_outer_pair(G1, ws1->ptr, G0, ws0->ptr, rt().stream());
    return w0;
  }
  sgd_matmul_(w1, g, h, true, false, alpha, b1);
  sgd_matmul_(w0, g0, x, true, false, alpha, b0);
  return w0;
}


TensorP pack_weight(const TensorP& wt) {
  if (wt->ndim != 2) fail("pack_weight: weights must be 2-D [out, in]");
  if (wt->dtype != DType::F16 && wt->dtype != DType::BF16) fail("pack_weight: fp16 or bf16 weights only");
  const int64_t N = wt->shape[0], K = wt->shape[1];
  TensorP out = alloc_out(wt->dtype, {(N + 15) / 16, (K + 31) / 32, 64, 8});
  LAUNCH k::pack_weights(wt->dtype, wt->data(), wt->strides[0], wt->strides[1], N, K, out->data(), rt().stream());
  return out;
}

TensorP pack_weight_x3(const TensorP& b) {
  if (b->ndim != 2) fail("pack_weight_x3: weights must be 2-D [in, out] (the B operand of x @ B)");
  if (b->dtype != DType::F32) fail("pack_weight_x3: fp32 weights only, got %s", dtype_name(b->dtype));
  const int64_t K = b->shape[0], N = b->shape[1];
  if (K % 16 != 0 || K == 0 || N == 0) fail("pack_weight_x3: the reduction dim %lld must be a positive multiple of 16", (long long)K);
  TensorP out = alloc_out(DType::BF16, {(N + 31) / 32, K / 16, 2, 64, 8});
  LAUNCH k::pack_weights_x3(b->data(), b->strides[0], b->strides[1], K, N, out->data(), rt().stream());
  return out;
}

bool is_x3_packed(const TensorP& t) {
  return t->ndim == 5 && t->dtype == DType::BF16 && t->shape[2] == 2 && t->shape[3] == 64 && t->shape[4] == 8;
}

TensorP pack_rows_x3(const TensorP& x) {
  if (x->ndim != 2) fail("pack_rows_x3: rows must be 2-D [rows, cols]");
  if (x->dtype != DType::F32) fail("pack_rows_x3: fp32 rows only, got %s", dtype_name(x->dtype));
  const int64_t M = x->shape[0], K = x->shape[1];
  if (K % 16 != 0 || K == 0 || M == 0)
    fail("pack_rows_x3: the column count %lld must be a positive multiple of 16", (long long)K);
  TensorP out = alloc_out(DType::BF16, {(M + 31) / 32, K / 16, 2, 64, 8});
  LAUNCH k::pack_rows_x3(x->data(), x->strides[0], x->strides[1], M, K, out->data(), rt().stream());
  return out;
}

// The packed-weight product.  a_rows < 0: a_in is fp32 [M, K]; otherwise a_in
// holds packed x3 rows of an [a_rows, K] matrix.
static TensorP matmul_x3(const TensorP& a_in, int64_t a_rows, const TensorP& pw, int64_t N, const Epilogue* epi,
                         PostLn* post_ln, PackOut* po) {
  const bool apk = a_rows >= 0;
  const char* name = apk ? "matmul_pp" : "matmul_packed";
  int64_t M, K;
  if (apk) {
    if (!is_x3_packed(a_in) || a_rows < 1 || a_in->shape[0] != (a_rows + 31) / 32)
      fail("%s: A must be pack_rows_x3 of [%lld, K] rows", name, (long long)a_rows);
    M = a_rows;
    K = a_in->shape[1] * 16;
  } else {
    if (a_in->ndim != 2) fail("%s: activations must be 2-D [rows, in]", name);
    if (a_in->dtype != DType::F32)
      fail("%s: fp32-packed weights take fp32 activations, got %s", name, dtype_name(a_in->dtype));
    M = a_in->shape[0];
    K = a_in->shape[1];
  }
  if (N < 1 || pw->shape[0] != (N + 31) / 32 || pw->shape[1] * 16 != K)
    fail("%s: packed weights hold [%lld/32, %lld/16] fragments, not [in %lld, out %lld]", name,
         (long long)pw->shape[0] * 32, (long long)pw->shape[1] * 16, (long long)K, (long long)N);
  // a layer_norm of A runs in the row-panel kernel's prologue when the plan
  // has one (fp32 gamma/beta [K]); otherwise as its own launch first
  if (epi && epi->ln_gamma) {
    if (apk) fail("%s: a layer_norm of packed rows is not available", name);
    if (!(k::gemm_x3_ln_ok(M, N, K) && epi->ln_beta && epi->ln_gamma->dtype == DType::F32 &&
          epi->ln_beta->dtype == DType::F32 && epi->ln_gamma->numel() == K && epi->ln_beta->numel() == K)) {
      Epilogue plain = *epi;
      plain.ln_gamma = plain.ln_beta = nullptr;
      return matmul_x3(layer_norm(a_in, epi->ln_gamma, epi->ln_beta, epi->ln_eps), -1, pw, N, &plain, post_ln, po);
    }
  }
  TensorP a = a_in;
  if (apk) a = contiguous(a_in);
  else if (!meta_mode() && (a->strides[1] != 1 || (M > 1 && a->strides[0] % 4 != 0) || ((uintptr_t)a->data() & 15)))
    a = materialize(a);
  TensorP pc = contiguous(pw);
  const std::vector<int64_t> od{M, N};
  const std::vector<int64_t> pkd{(M + 31) / 32, N / 16, 2, 64, 8};
  // packed rows and row statistics straight from a row-panel epilogue when
  // the plan has one (unsplit, or split with its tiles finished in the launch)
  const bool panel = !post_ln && k::gemm_x3_rows_out_ok(M, N, K, apk);
  const bool pk_direct = po && po->want_pk && panel && N % 16 == 0;
  const bool st_direct = po && po->want_stats && panel && N % 32 == 0;
  const bool norm = epi && epi->norm_stats;
  if (norm && !(apk && k::gemm_x3_panel_ok(M, N, K, true)))
    fail("%s: a folded layer_norm needs packed rows and a row-panel plan (K = 256..1536 in steps of 256)", name);
  const bool want_c = !po || po->want_c || (po->want_pk && !pk_direct) || (po->want_stats && !st_direct);
  TensorP out = want_c ? alloc_out(DType::F32, od) : nullptr;
  k::Gemm g;
  g.dt = g.b_dt = DType::F32;
  g.M = M; g.N = N; g.K = K; g.batch = 1;
  g.A = a->data();
  if (apk) {
    g.a_x3 = true;
  } else {
    g.a_sm = M == 1 ? K : a->strides[0];
    g.a_sk = 1;
  }
  g.B = pc->data(); g.b_x3 = true;
  g.C = out ? out->data() : nullptr; g.c_sm = N; g.c_sb = M * N;
  if (pk_direct) {
    po->pk = alloc_out(DType::BF16, pkd);
    g.c_pk = po->pk->data();
  }
  if (st_direct) {
    po->stats = alloc_out(DType::F32, {M, N / 32, 2});
    g.rs_out = (float*)po->stats->data();
  }
  TensorP nst, ncs;
  if (norm) {
    if (!epi->norm_cs || epi->norm_stats->dtype != DType::F32 || epi->norm_cs->dtype != DType::F32 ||
        epi->norm_stats->ndim != 3 || epi->norm_stats->shape[0] != M || epi->norm_stats->shape[1] * 32 != K ||
        epi->norm_stats->shape[2] != 2 || epi->norm_cs->numel() != N)
      fail("%s: layer_norm statistics must be row_stats_x3 of the [%lld, %lld] rows and cs [%lld] fp32", name,
           (long long)M, (long long)K, (long long)N);
    nst = contiguous(epi->norm_stats);
    ncs = contiguous(epi->norm_cs);
    g.rs_in = (const float*)nst->data();
    g.rs_cs = (const float*)ncs->data();
    g.rs_tiles = (int)(K / 32);
    g.rs_n = K;
    g.rs_eps = epi->norm_eps;
  }
  EpiKeep keep;
  set_epilogue(g, epi, od, {}, &keep);
  TensorP pl_g, pl_b;
  bool pln_fused = false;
  if (post_ln) {
    if (!post_ln->gamma || !post_ln->beta || post_ln->gamma->dtype != g.dt || post_ln->beta->dtype != g.dt ||
        post_ln->gamma->numel() != N || post_ln->beta->numel() != N)
      fail("%s: layer_norm gamma and beta must be [%lld] of the output dtype", name, (long long)N);
    if (post_ln->want_pk && N % 16 != 0) fail("%s: packed layer_norm rows need N %% 16 == 0", name);
    pl_g = contiguous(post_ln->gamma);
    pl_b = contiguous(post_ln->beta);
    if (!meta_mode()) {
      TensorP y = post_ln->want_y ? alloc_out(g.dt, od) : nullptr;
      TensorP ypk = post_ln->want_pk ? alloc_out(DType::BF16, pkd) : nullptr;
      k::Gemm probe = g;
      probe.pln_gamma = pl_g->data();
      probe.pln_beta = pl_b->data();
      probe.pln_y = y ? y->data() : nullptr;
      probe.pln_ypk = ypk ? ypk->data() : nullptr;
      probe.pln_eps = post_ln->eps;
      pln_fused = k::gemm_post_ln_fused(probe);
      if (pln_fused) {
        g = probe;
        post_ln->y = y;
        post_ln->ypk = ypk;
      }
    }
  }
  if (!meta_mode() && !k::gemm_x3_ok(g)) fail("%s: this product cannot use the packed fp32 weights", name);
  const size_t wsb = meta_mode() ? 0 : k::gemm_workspace_bytes(g);
  BufferP ws;
  if (wsb) ws = scratch(wsb);
  LAUNCH k::gemm(g, ws ? ws->ptr : nullptr, rt().stream());
  if (post_ln && !pln_fused) {
    TensorP y = layer_norm(out, pl_g, pl_b, post_ln->eps);
    if (post_ln->want_y) post_ln->y = y;
    if (post_ln->want_pk) post_ln->ypk = pack_rows_x3(y);
  }
  if (po && po->want_pk && !pk_direct) po->pk = pack_rows_x3(out);
  if (po && po->want_stats && !st_direct) po->stats = row_stats_x3(out);
  return po && !po->want_c ? nullptr : out;
}

TensorP row_stats_x3(const TensorP& x) {
  if (x->ndim != 2 || x->dtype != DType::F32) fail("row_stats_x3: fp32 [rows, cols] expected");
  const int64_t M = x->shape[0], N = x->shape[1];
  if (N % 32 != 0 || N == 0) fail("row_stats_x3: the column count %lld must be a positive multiple of 32", (long long)N);
  TensorP a = x;
  if (!meta_mode() && (a->strides[1] != 1 || a->strides[0] % 4 != 0 || ((uintptr_t)a->data() & 15))) a = materialize(a);
  TensorP out = alloc_out(DType::F32, {M, N / 32, 2});
  LAUNCH k::row_tile_stats((const float*)a->data(), M == 1 ? N : a->strides[0], M, N, (float*)out->data(),
                           rt().stream());
  return out;
}

TensorP matmul_pp_norm(const TensorP& apk, const TensorP& stats, int64_t M, const TensorP& folded,
                       const TensorP& cs, int64_t N, float eps, const Epilogue* epi, PackOut* po) {
  Epilogue e = epi ? *epi : Epilogue{};
  e.norm_stats = stats;
  e.norm_cs = cs;
  e.norm_eps = eps;
  return matmul_pp(apk, M, folded, N, &e, nullptr, po);
}

TensorP matmul_pp(const TensorP& apk, int64_t M, const TensorP& pw, int64_t N, const Epilogue* epi, PostLn* post_ln,
                  PackOut* po) {
  if (!is_x3_packed(pw)) fail("matmul_pp: weights must be packed by pack_weight_x3");
  if (M < 0) fail("matmul_pp: negative row count");
  return matmul_x3(apk, M, pw, N, epi, post_ln, po);
}

TensorP matmul_packed(const TensorP& a_in, const TensorP& pw, int64_t N, const Epilogue* epi, PostLn* post_ln,
                      PackOut* po) {
  if (is_x3_packed(pw)) return matmul_x3(a_in, -1, pw, N, epi, post_ln, po);
  if (post_ln || po) fail("matmul_packed: layer_norm or packed rows of the output need the fp32 packed layout");
  const char* name = "matmul_packed";
  if (a_in->ndim != 2) fail("%s: activations must be 2-D [rows, in]", name);
  if (pw->ndim != 4 || pw->shape[2] != 64 || pw->shape[3] != 8) fail("%s: weights are not packed (pack_weight)", name);
  if (a_in->dtype != pw->dtype) fail("Dtype mismatch: %s vs %s", dtype_name(a_in->dtype), dtype_name(pw->dtype));
  const int64_t M = a_in->shape[0], K = a_in->shape[1];
  if (N < 1 || pw->shape[0] != (N + 15) / 16 || pw->shape[1] != (K + 31) / 32)
    fail("%s: packed weights hold [%lld/16, %lld/32] tiles, not [out %lld, in %lld]", name,
         (long long)pw->shape[0] * 16, (long long)pw->shape[1] * 32, (long long)N, (long long)K);
  TensorP a = a_in;
  if (!meta_mode() && (a->strides[1] != 1 || (M > 1 && a->strides[0] % 8 != 0) || ((uintptr_t)a->data() & 15)))
    a = materialize(a);
  TensorP pc = contiguous(pw);
  const std::vector<int64_t> od{M, N};
  TensorP out = alloc_out(a->dtype, od);
  k::Gemm g;
  g.dt = g.b_dt = a->dtype;
  g.M = M; g.N = N; g.K = K; g.batch = 1;
  g.A = a->data(); g.a_sm = M == 1 ? K : a->strides[0]; g.a_sk = 1;
  g.B = pc->data(); g.b_packed = true; g.b_sk = 1; g.b_sn = K;
  g.C = out->data(); g.c_sm = N; g.c_sb = M * N;
  EpiKeep keep;
  set_epilogue(g, epi, od, {}, &keep);
  if (!meta_mode() && !k::gemm_is_skinny(g))
    fail("%s: needs at most 16 fp16/bf16 rows with the reduction dim a multiple of 8", name);
  if (epi && epi->ln_gamma && !meta_mode() && !k::gemm_skinny_ln_ok(g)) {
    Epilogue plain = *epi;
    plain.ln_gamma = plain.ln_beta = nullptr;
    return matmul_packed(layer_norm(a_in, epi->ln_gamma, epi->ln_beta, epi->ln_eps), pw, N, &plain);
  }
  LAUNCH k::gemm(g, nullptr, rt().stream());
  return out;
}

TensorP linear_int8(const TensorP& x, const TensorP& q, const TensorP& scale) {
  check_dtype("linear_int8", kFloatOnly, x->dtype);
  if (q->dtype != DType::I8 || q->ndim != 2) fail("linear_int8: weights must be 2-D int8");
  if (scale->dtype != DType::F32 || scale->numel() != q->shape[0]) fail("linear_int8: scales must be f32 [out]");
  if (x->shape[x->ndim - 1] != q->shape[1]) fail("linear_int8: inner dimension mismatch");
  TensorP xc = contiguous(x), qc = contiguous(q), sc = contiguous(scale);
  const int64_t K = q->shape[1], N = q->shape[0];
  const int64_t M = xc->numel() / K;
  std::vector<int64_t> od = xc->dims();
  od.back() = N;
  TensorP out = alloc_out(x->dtype, od);
  k::Gemm g;
  g.dt = x->dtype; g.b_dt = DType::I8;
  g.M = M; g.N = N; g.K = K; g.batch = 1;
  g.A = xc->data(); g.a_sm = K; g.a_sk = 1;
  g.B = qc->data(); g.b_sk = 1; g.b_sn = K;
  g.b_scale = (const float*)sc->data();
  g.C = out->data(); g.c_sm = N;
  size_t wsb = meta_mode() ? 0 : k::gemm_workspace_bytes(g);
  BufferP ws;
  if (wsb) ws = scratch(wsb);
  LAUNCH k::gemm(g, ws ? ws->ptr : nullptr, rt().stream());
  return out;
}

// ── attention ──────────────────────────────────────────────────────────────
TensorP attention(const TensorP& q, const TensorP& kk, const TensorP& v, bool causal, bool out_layout_thd,
                  float scale_arg) {
  const char* name = causal ? "attention_causal" : "attention";
  if (q->ndim < 2 || kk->ndim < 2 || v->ndim < 2) fail("%s requires at least 2D tensors for Q, K, V", name);
  check_dtype(name, kFloatOnly, q->dtype);
  if (q->dtype != kk->dtype || q->dtype != v->dtype) fail("%s: Q, K, V dtypes differ", name);
  const int64_t D = q->shape[q->ndim - 1];
  if (kk->shape[kk->ndim - 1] != D)
    fail("Q and K must have same d_k: %lld vs %lld", (long long)D, (long long)kk->shape[kk->ndim - 1]);
  const int64_t Tk = kk->shape[kk->ndim - 2];
  if (v->shape[v->ndim - 2] != Tk)
    fail("K and V must have same kv_len: %lld vs %lld", (long long)Tk, (long long)v->shape[v->ndim - 2]);
  const int64_t Dv = v->shape[v->ndim - 1];
  const int64_t Tq = q->shape[q->ndim - 2];
  if (scale_arg < 0.f || !std::isfinite(scale_arg)) fail("%s: scale must be finite and >= 0", name);
  const float scale = scale_arg > 0.f ? scale_arg : 1.0f / std::sqrt((float)D);
  std::vector<int64_t> lead(q->shape, q->shape + q->ndim - 2);
  bool same_lead = q->ndim == kk->ndim && q->ndim == v->ndim;
  for (int i = 0; same_lead && i < q->ndim - 2; ++i)
    same_lead = kk->shape[i] == q->shape[i] && v->shape[i] == q->shape[i];

  k::Attn a;
  a.dt = q->dtype;
  a.Tq = Tq; a.Tk = Tk; a.D = D;
  a.causal = causal;
  a.scale = scale;
  bool fused = same_lead && Dv == D && k::attention_supported(a) && q->ndim <= 4 &&
               q->strides[q->ndim - 1] == 1 && kk->strides[kk->ndim - 1] == 1 && v->strides[v->ndim - 1] == 1;
  if (!fused) {
    // Composition, as the reference records it: Q K^T, scale, softmax, @ V.
    Epilogue e;
    e.alpha = scale;
    TensorP s = matmul(q, kk, false, true, &e);
    TensorP p = softmax(s, causal ? k::kSoftmaxCausal : k::kSoftmax);
    return matmul(p, v);
  }
  // leading dims -> (B, H)
  auto lead_strides = [](const Tensor& t, int64_t* sb, int64_t* sh) {
    if (t.ndim == 2) { *sb = 0; *sh = 0; }
    else if (t.ndim == 3) { *sb = 0; *sh = t.strides[0]; }
    else { *sb = t.strides[0]; *sh = t.strides[1]; }
  };
  a.B = q->ndim == 4 ? q->shape[0] : 1;
  a.H = q->ndim == 4 ? q->shape[1] : (q->ndim == 3 ? q->shape[0] : 1);
  a.q = q->data(); lead_strides(*q, &a.q_sb, &a.q_sh); a.q_st = q->strides[q->ndim - 2];
  a.k = kk->data(); lead_strides(*kk, &a.k_sb, &a.k_sh); a.k_st = kk->strides[kk->ndim - 2];
  a.v = v->data(); lead_strides(*v, &a.v_sb, &a.v_sh); a.v_st = v->strides[v->ndim - 2];
  std::vector<int64_t> od = q->dims();
  TensorP out;
  if (out_layout_thd && q->ndim >= 3) {
    // physical [B, T, H, D]; logical [B, H, T, D]
    std::vector<int64_t> phys;
    if (q->ndim == 4) phys = {a.B, Tq, a.H, D};
    else phys = {Tq, a.H, D};
    TensorP base = alloc_out(q->dtype, phys);
    out = make_meta(q->dtype, od);
    out->buf = base->buf;
    out->offset = base->offset;
    if (q->ndim == 4) {
      out->strides[0] = Tq * a.H * D; out->strides[1] = D; out->strides[2] = a.H * D; out->strides[3] = 1;
    } else {
      out->strides[0] = D; out->strides[1] = a.H * D; out->strides[2] = 1;
    }
  } else {
    out = alloc_out(q->dtype, od);
  }
  a.o = out->data();
  lead_strides(*out, &a.o_sb, &a.o_sh);
  a.o_st = out->strides[out->ndim - 2];
  LAUNCH k::attention(a, rt().stream());
  return out;
}

TensorP attention_rows_x3(const TensorP& q, const TensorP& kk, const TensorP& v, bool causal, float scale_arg) {
  if (q->ndim < 3 || q->ndim > 4 || kk->ndim != q->ndim || v->ndim != q->ndim) return nullptr;
  if (q->dtype != DType::F32 || kk->dtype != DType::F32 || v->dtype != DType::F32) return nullptr;
  for (int i = 0; i < q->ndim - 2; ++i)
    if (kk->shape[i] != q->shape[i] || v->shape[i] != q->shape[i]) return nullptr;
  const int64_t D = q->shape[q->ndim - 1], Tq = q->shape[q->ndim - 2], Tk = kk->shape[kk->ndim - 2];
  if (kk->shape[kk->ndim - 1] != D || v->shape[v->ndim - 1] != D || v->shape[v->ndim - 2] != Tk) return nullptr;
  if (q->strides[q->ndim - 1] != 1 || kk->strides[kk->ndim - 1] != 1 || v->strides[v->ndim - 1] != 1) return nullptr;
  if (scale_arg < 0.f || !std::isfinite(scale_arg)) return nullptr;
  k::Attn a;
  a.dt = DType::F32;
  a.Tq = Tq; a.Tk = Tk; a.D = D;
  a.causal = causal;
  a.scale = scale_arg > 0.f ? scale_arg : 1.0f / std::sqrt((float)D);
  if (!k::attention_supported(a)) return nullptr;
  a.B = q->ndim == 4 ? q->shape[0] : 1;
  a.H = q->ndim == 4 ? q->shape[1] : q->shape[0];
  if ((a.H * D) % 16 != 0) return nullptr;
  auto lead = [](const Tensor& t, int64_t* sb, int64_t* sh) {
    if (t.ndim == 3) { *sb = 0; *sh = t.strides[0]; }
    else { *sb = t.strides[0]; *sh = t.strides[1]; }
  };
  a.q = q->data(); lead(*q, &a.q_sb, &a.q_sh); a.q_st = q->strides[q->ndim - 2];
  a.k = kk->data(); lead(*kk, &a.k_sb, &a.k_sh); a.k_st = kk->strides[kk->ndim - 2];
  a.v = v->data(); lead(*v, &a.v_sb, &a.v_sh); a.v_st = v->strides[v->ndim - 2];
  const int64_t rows = a.B * Tq;
  TensorP out = alloc_out(DType::BF16, {(rows + 31) / 32, a.H * D / 16, 2, 64, 8});
  a.o_pk = out->data();
  LAUNCH k::attention(a, rt().stream());
  return out;
}

TensorP qkv_attention(const TensorP& x, const TensorP& w, const TensorP& b, int64_t n_head, bool causal,
                      int64_t batch, bool read_partials) {
  const char* name = "qkv_attention";
  // w is [K, 3d], or the same weights packed by pack_weight_x3 (fp32)
  const bool x3 = is_x3_packed(w);
  if (x->ndim != 2 || (w->ndim != 2 && !x3) || b->ndim != 1)
    fail("%s: x [B*T, K], w [K, 3d] (or its pack_weight_x3 packing) and b [3d] expected", name);
  check_dtype(name, kFloatOnly, x->dtype);
  if ((!x3 && w->dtype != x->dtype) || b->dtype != x->dtype || (x3 && x->dtype != DType::F32))
    fail("%s: dtypes differ", name);
  const int64_t R = x->shape[0], K = x->shape[1], N = x3 ? b->numel() : w->shape[1];
  if ((x3 ? (w->shape[0] != (N + 31) / 32 || w->shape[1] * 16 != K) : w->shape[0] != K) || b->numel() != N ||
      N % 3 != 0)
    fail("%s: w must be [%lld, 3d] and b [3d]", name, (long long)K);
  const int64_t d = N / 3;
  if (n_head <= 0 || d % n_head != 0) fail("%s: %lld columns do not split into %lld heads", name, (long long)d,
                                           (long long)n_head);
  if (batch <= 0 || R % batch != 0) fail("%s: %lld rows do not split into %lld sequences", name, (long long)R,
                                         (long long)batch);
  const int64_t T = R / batch, hd = d / n_head;

  // The composed path: one GEMM with the bias, head views, attention.
  auto composed = [&]() {
    Epilogue e;
    e.bias = b;
    TensorP qkv = x3 ? matmul_packed(x, w, N, &e) : matmul(x, w, false, false, &e);
    auto heads = [&](int64_t lo) {
      TensorP part = slice(qkv, 1, lo, lo + d);
      return transpose_dims(reshape(part, {batch, T, n_head, hd}), 1, 2);
    };
    TensorP a = attention(heads(0), heads(d), heads(2 * d), causal, true);
    return reshape(transpose_dims(a, 1, 2), {R, d});
  };
  if (meta_mode() || !read_partials || x->dtype != DType::F32) return composed();

  TensorP xc = x;
  if (x->strides[1] != 1 || (x3 && ((R > 1 && x->strides[0] % 4 != 0) || ((uintptr_t)x->data() & 15))))
    xc = materialize(x);
  TensorP wc = x3 || w->strides[1] == 1 ? w : contiguous(w);
  TensorP bc = contiguous(b);
  k::Gemm g;
  g.dt = g.b_dt = DType::F32;
  g.M = R; g.N = N; g.K = K; g.batch = 1;
  g.A = xc->data(); g.a_sm = R == 1 ? K : xc->strides[0]; g.a_sk = 1; g.a_sb = R * K;
  g.B = wc->data();
  if (x3) {
    g.b_x3 = true;
  } else {
    g.b_sk = wc->strides[0]; g.b_sn = 1; g.b_sb = K * N;
  }
  g.C = nullptr; g.c_sm = N; g.c_sb = R * N;
  g.no_reduce = true;
  if (x3 && !k::gemm_x3_ok(g)) return composed();
  const int splits = k::gemm_splits(g);
  k::Attn a;
  a.dt = DType::F32;
  a.B = batch; a.H = n_head; a.Tq = T; a.Tk = T; a.D = hd;
  a.causal = causal;
  a.scale = 1.0f / std::sqrt((float)hd);
  a.q_sb = a.k_sb = a.v_sb = T * N;
  a.q_sh = a.k_sh = a.v_sh = hd;
  a.q_st = a.k_st = a.v_st = N;
  a.nsplit = splits;
  a.plane = R * N;
  a.b_sh = hd;
  if (!(splits == 2 || splits == 4 || splits == 8)) return composed();
  BufferP ws = scratch(k::gemm_workspace_bytes(g));
  float* w0 = (float*)ws->ptr;
  a.q = w0; a.k = w0 + d; a.v = w0 + 2 * d;
  a.qb = bc->data(); a.kb = (const float*)bc->data() + d; a.vb = (const float*)bc->data() + 2 * d;
  TensorP out = alloc_out(DType::F32, {batch, T, n_head, hd});
  a.o = out->data();
  a.o_sb = T * d; a.o_sh = hd; a.o_st = d;
  if (!k::attention_partials_ok(a)) return composed();
  LAUNCH k::gemm(g, ws->ptr, rt().stream());
  LAUNCH k::attention(a, rt().stream());
  return reshape(out, {R, d});
}

// ── KV-cache decode ────────────────────────────────────────────────────────
// Shape checks shared by kv_write and decode_attention: 4-D [B, H, T, D]
// operands with a unit stride along D.
static void check_bhtd(const char* name, const char* what, const Tensor& t) {
  if (t.ndim != 4) fail("%s: %s must be 4-D [batch, heads, tokens, head_dim], got %s", name, what,
                        shape_str(t.dims()).c_str());
  if (t.strides[3] != 1 && t.shape[3] > 1) fail("%s: %s must have a unit stride along head_dim", name, what);
}

static TensorP check_lens(const char* name, const char* what, const TensorP& lens, int64_t B) {
  if (lens->dtype != DType::I32) fail("%s: %s must be int32, got %s", name, what, dtype_name(lens->dtype));
  if (lens->numel() != B) fail("%s: %s must hold one entry per sequence (%lld), got %lld", name, what,
                               (long long)B, (long long)lens->numel());
  return contiguous(lens);
}

TensorP decode_attention(const TensorP& q, const TensorP& kc, const TensorP& vc, const TensorP& lens,
                         const TensorP& k_new, const TensorP& v_new) {
  const char* name = "decode_attention";
  check_dtype(name, kFloatOnly, q->dtype);
  if (kc->dtype != q->dtype || vc->dtype != q->dtype) fail("%s: q and the caches must share a dtype", name);
  check_bhtd(name, "q", *q);
  check_bhtd(name, "k_cache", *kc);
  check_bhtd(name, "v_cache", *vc);
  const int64_t B = q->shape[0], H = q->shape[1], Tq = q->shape[2], D = q->shape[3];
  for (const Tensor* c : {kc.get(), vc.get()})
    if (c->shape[0] != B || c->shape[1] != H || c->shape[3] != D)
      fail("%s: cache shape %s does not match q %s", name, shape_str(c->dims()).c_str(), shape_str(q->dims()).c_str());
  if (vc->shape[2] != kc->shape[2]) fail("%s: k_cache and v_cache lengths differ", name);
  const int64_t Tmax = kc->shape[2];
  if (Tmax < 1) fail("%s: empty cache", name);
  if (Tq > Tmax) fail("%s: %lld query rows exceed the cache length %lld", name, (long long)Tq, (long long)Tmax);
  TensorP lc = check_lens(name, "lens", lens, B);

  k::DecodeAttn a;
  a.dt = q->dtype;
  a.B = B; a.H = H; a.Tq = Tq; a.Tmax = Tmax; a.D = D;
  if (!k::decode_attention_supported(a)) fail("%s: head dim %lld not supported (32, 64 or 128)", name, (long long)D);
  a.scale = 1.0f / std::sqrt((float)D);
  a.q = q->data(); a.q_sb = q->strides[0]; a.q_sh = q->strides[1]; a.q_st = q->strides[2];
  a.k = kc->data(); a.k_sb = kc->strides[0]; a.k_sh = kc->strides[1]; a.k_st = kc->strides[2];
  a.v = vc->data(); a.v_sb = vc->strides[0]; a.v_sh = vc->strides[1]; a.v_st = vc->strides[2];
  a.lens = (const int32_t*)lc->data();
  if (k_new || v_new) {
    if (!k_new || !v_new) fail("%s: new K and V rows come together", name);
    if (Tq != 1) fail("%s: appending new rows needs one query row per sequence, got %lld", name, (long long)Tq);
    for (const TensorP& t : {k_new, v_new}) {
      if (t->dtype != q->dtype) fail("%s: new rows must share q's dtype", name);
      check_bhtd(name, "new rows", *t);
      if (t->shape[0] != B || t->shape[1] != H || t->shape[2] != 1 || t->shape[3] != D)
        fail("%s: new rows must be [%lld, %lld, 1, %lld]", name, (long long)B, (long long)H, (long long)D);
    }
    a.kn = k_new->data(); a.kn_sb = k_new->strides[0]; a.kn_sh = k_new->strides[1];
    a.vn = v_new->data(); a.vn_sb = v_new->strides[0]; a.vn_sh = v_new->strides[1];
  }
  // physical [B, Tq, H, D], logical [B, H, Tq, D]
  TensorP base = alloc_out(q->dtype, {B, Tq, H, D});
  TensorP out = make_meta(q->dtype, q->dims());
  out->buf = base->buf;
  out->offset = base->offset;
  out->strides[0] = Tq * H * D; out->strides[1] = D; out->strides[2] = H * D; out->strides[3] = 1;
  a.o = out->data(); a.o_sb = out->strides[0]; a.o_sh = out->strides[1]; a.o_st = out->strides[2];
  size_t wsb = meta_mode() ? 0 : k::decode_attention_ws_bytes(a);
  BufferP ws;
  if (wsb) ws = scratch(wsb);
  LAUNCH k::decode_attention(a, ws ? ws->ptr : nullptr, rt().stream());
  return out;
}

static void check_kv_pair(const char* name, const TensorP& cache, const TensorP& rows) {
  if (cache->dtype != rows->dtype) fail("%s: cache is %s but rows are %s", name, dtype_name(cache->dtype),
                                        dtype_name(rows->dtype));
  check_bhtd(name, "cache", *cache);
  check_bhtd(name, "rows", *rows);
  if (rows->shape[0] != cache->shape[0] || rows->shape[1] != cache->shape[1] || rows->shape[3] != cache->shape[3])
    fail("%s: rows %s do not match cache %s", name, shape_str(rows->dims()).c_str(), shape_str(cache->dims()).c_str());
  if (rows->shape[2] > cache->shape[2]) fail("%s: %lld rows exceed the cache length %lld", name,
                                             (long long)rows->shape[2], (long long)cache->shape[2]);
  for (int i = 0; i < 3; ++i)
    if (cache->shape[i] > 1 && cache->strides[i] == 0) fail("%s: cache has overlapping rows", name);
}

void kv_write(const TensorP& cache, const TensorP& rows, const TensorP& pos, const TensorP& cache2,
              const TensorP& rows2) {
  const char* name = "kv_write";
  check_kv_pair(name, cache, rows);
  if (cache2) {
    check_kv_pair(name, cache2, rows2);
    if (cache2->dims() != cache->dims() || rows2->dims() != rows->dims() || cache2->dtype != cache->dtype)
      fail("%s: the two caches (and their rows) must have the same shape and dtype", name);
  }
  const int64_t B = cache->shape[0];
  TensorP pc = check_lens(name, "positions", pos, B);
  k::KvWrite a;
  a.dt = cache->dtype;
  a.B = B; a.H = cache->shape[1]; a.T = rows->shape[2]; a.D = cache->shape[3]; a.Tmax = cache->shape[2];
  a.cache = cache->data(); a.src = rows->data();
  for (int i = 0; i < 3; ++i) { a.cs[i] = cache->strides[i]; a.xs[i] = rows->strides[i]; }
  if (cache2) {
    a.cache2 = cache2->data(); a.src2 = rows2->data();
    for (int i = 0; i < 3; ++i) { a.c2s[i] = cache2->strides[i]; a.x2s[i] = rows2->strides[i]; }
  }
  a.pos = (const int32_t*)pc->data();
  LAUNCH k::kv_write(a, rt().stream());
}

}  // namespace ops
}  // namespace agpu
