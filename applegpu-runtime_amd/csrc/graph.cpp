// Op table, eager/lazy op runner and the lazy graph executor.
#include "graph.hpp"

#include <cmath>
#include <unordered_map>
#include <unordered_set>

#include "ops.hpp"

namespace agpu {

// ── meta mode ──────────────────────────────────────────────────────────────
static thread_local bool t_meta = false;
bool meta_mode() { return t_meta; }
MetaScope::MetaScope() : prev(t_meta) { t_meta = true; }
MetaScope::~MetaScope() { t_meta = prev; }

// ── op table ───────────────────────────────────────────────────────────────
// Names follow the Python surface of the reference (crates/python/src/lib.rs).
enum Op : int {
  OP_ADD, OP_SUB, OP_MUL, OP_DIV, OP_MIN, OP_MAX, OP_MOD, OP_AND, OP_OR, OP_XOR,
  OP_LT, OP_GT, OP_LE, OP_GE, OP_EQ, OP_NE,
  OP_NEG, OP_RELU, OP_EXP, OP_LOG, OP_SQRT, OP_ABS, OP_SIGN, OP_TANH, OP_SIN, OP_COS, OP_SIGMOID,
  OP_GELU, OP_GELU_EXACT, OP_LOGICAL_NOT, OP_BITWISE_NOT,
  OP_SCALAR_MUL, OP_POW, OP_CLAMP, OP_SHL, OP_SHR, OP_CAST, OP_QUANTIZE, OP_DEQUANTIZE,
  OP_SOFTMAX, OP_LOG_SOFTMAX, OP_SOFTMAX_CAUSAL, OP_LAYER_NORM,
  OP_SUM, OP_MEAN, OP_AMAX, OP_ARGMAX, OP_VAR, OP_STD,
  OP_SUM_DIM, OP_MEAN_ALL, OP_MSE_LOSS, OP_MSE_LOSS_BACKWARD, OP_SOFTMAX_BACKWARD, OP_THRESHOLD_BACKWARD,
  OP_EMBEDDING, OP_INDEX_SELECT, OP_GATHER, OP_CONCAT, OP_SLICE, OP_RESHAPE, OP_TRANSPOSE, OP_TRANSPOSE_DIMS,
  OP_MATMUL, OP_MATMUL_EX, OP_LINEAR, OP_ADD_BIAS, OP_ATTENTION, OP_ATTENTION_CAUSAL,
  OP_WHERE, OP_MASKED_FILL, OP_TRIU, OP_TRIL,
  OP_QUANTIZE_PER_ROW, OP_DEQUANTIZE_PER_ROW, OP_LINEAR_INT8, OP_CONTIGUOUS, OP_FULL,
  OP_DECODE_ATTENTION, OP_PACK_WEIGHT, OP_MATMUL_PACKED,
  OP_SGD_MATMUL, OP_SGD_SUM_ROWS, OP_MSE_LOSS_GRAD, OP_QKV_ATTENTION,
  OP_LAYER_NORM_BACKWARD, OP_LAYER_NORM_GRADS, OP_GELU_BACKWARD, OP_GELU_TANH_BACKWARD, OP_GELU_EXACT_BACKWARD,
  OP_EMBEDDING_BACKWARD, OP_PACK_WEIGHT_X3, OP_PACK_ROWS_X3, OP_MATMUL_PP, OP_ROW_STATS_X3, OP_MATMUL_PP_NORM,
  OP_LINEAR_BACKWARD_SGD, OP_LINEAR_MSE_BACKWARD_SGD, OP_MLP2_SGD_STEP, OP_LINEAR_BACKWARD_SGD_PAIR,
  OP_LINEAR_RELU_MSE_BACKWARD_SGD,
  OP_COUNT
};

static const char* kNames[OP_COUNT] = {
    "add", "sub", "mul", "div", "elem_min", "elem_max", "mod", "bitwise_and", "bitwise_or", "bitwise_xor",
    "lt", "gt", "le", "ge", "eq", "ne",
    "neg", "relu", "exp", "log", "sqrt", "abs", "sign", "tanh", "sin", "cos", "sigmoid",
    "gelu", "gelu_exact", "logical_not", "bitwise_not",
    "scalar_mul", "pow", "clamp", "shl", "shr", "cast", "quantize", "dequantize",
    "softmax", "log_softmax", "softmax_causal", "layer_norm",
    "sum", "mean", "amax", "argmax", "var", "std",
    "sum_dim", "mean_all", "mse_loss", "mse_loss_backward", "softmax_backward", "threshold_backward",
    "embedding", "index_select", "gather", "concat", "slice", "reshape", "transpose", "transpose_dims",
    "matmul", "matmul_ex", "linear", "add_bias", "attention", "attention_causal",
    "where", "masked_fill", "triu", "tril",
    "quantize_per_row", "dequantize_per_row", "linear_int8", "contiguous", "full",
    "decode_attention", "pack_weight", "matmul_packed",
    "sgd_matmul_", "sgd_sum_rows_", "mse_loss_grad", "qkv_attention",
    "layer_norm_backward", "layer_norm_grads", "gelu_backward", "gelu_tanh_backward", "gelu_exact_backward",
    "embedding_backward", "pack_weight_x3", "pack_rows_x3", "matmul_pp", "row_stats_x3", "matmul_pp_norm",
    "linear_backward_sgd_", "linear_mse_backward_sgd_", "mlp2_sgd_step_", "linear_backward_sgd_pair_",
    "linear_relu_mse_backward_sgd_",
};

int op_code(const char* name) {
  static std::unordered_map<std::string, int> m = [] {
    std::unordered_map<std::string, int> r;
    for (int i = 0; i < OP_COUNT; ++i) r[kNames[i]] = i;
    r["mod_"] = OP_MOD;
    r["eq_"] = OP_EQ;
    r["ne_"] = OP_NE;
    r["std_dev"] = OP_STD;
    r["where_cond"] = OP_WHERE;
    return r;
  }();
  auto it = m.find(name);
  return it == m.end() ? -1 : it->second;
}
const char* op_name(int code) { return code >= 0 && code < OP_COUNT ? kNames[code] : "?"; }
int op_outputs(int code) {
  if (code == OP_LAYER_NORM_GRADS) return 3;
  return code == OP_QUANTIZE_PER_ROW || code == OP_MSE_LOSS_GRAD ? 2 : 1;
}

static void need(const std::vector<TensorP>& in, size_t n, int code) {
  if (in.size() != n) fail("%s expects %zu tensor inputs, got %zu", op_name(code), n, in.size());
}
static double fp(const std::vector<double>& f, size_t i, int code) {
  if (i >= f.size()) fail("%s: missing float parameter %zu", op_name(code), i);
  return f[i];
}
static int64_t ip(const std::vector<int64_t>& v, size_t i, int code) {
  if (i >= v.size()) fail("%s: missing integer parameter %zu", op_name(code), i);
  return v[i];
}
static DType dt_param(int64_t w) {
  DType d;
  if (!dtype_from_wire((int)w, &d)) fail("invalid dtype wire value: %lld", (long long)w);
  return d;
}

std::vector<TensorP> run_op(int code, const std::vector<TensorP>& in, const std::vector<double>& f,
                            const std::vector<int64_t>& iv) {
  using namespace ops;
  switch (code) {
    case OP_ADD: case OP_SUB: case OP_MUL: case OP_DIV: case OP_MIN: case OP_MAX: case OP_MOD:
    case OP_AND: case OP_OR: case OP_XOR: case OP_LT: case OP_GT: case OP_LE: case OP_GE: case OP_EQ:
    case OP_NE:
      need(in, 2, code);
      return {binary(code - OP_ADD, in[0], in[1])};
    case OP_NEG: return need(in, 1, code), std::vector<TensorP>{unary(k::kNeg, in[0])};
    case OP_RELU: return need(in, 1, code), std::vector<TensorP>{unary(k::kRelu, in[0])};
    case OP_EXP: return need(in, 1, code), std::vector<TensorP>{unary(k::kExp, in[0])};
    case OP_LOG: return need(in, 1, code), std::vector<TensorP>{unary(k::kLog, in[0])};
    case OP_SQRT: return need(in, 1, code), std::vector<TensorP>{unary(k::kSqrt, in[0])};
    case OP_ABS: return need(in, 1, code), std::vector<TensorP>{unary(k::kAbs, in[0])};
    case OP_SIGN: return need(in, 1, code), std::vector<TensorP>{unary(k::kSign, in[0])};
    case OP_TANH: return need(in, 1, code), std::vector<TensorP>{unary(k::kTanh, in[0])};
    case OP_SIN: return need(in, 1, code), std::vector<TensorP>{unary(k::kSin, in[0])};
    case OP_COS: return need(in, 1, code), std::vector<TensorP>{unary(k::kCos, in[0])};
    case OP_SIGMOID: return need(in, 1, code), std::vector<TensorP>{unary(k::kSigmoid, in[0])};
    case OP_GELU: return need(in, 1, code), std::vector<TensorP>{unary(k::kGelu, in[0])};
    case OP_GELU_EXACT: return need(in, 1, code), std::vector<TensorP>{unary(k::kGeluExact, in[0])};
    case OP_LOGICAL_NOT: return need(in, 1, code), std::vector<TensorP>{unary(k::kLogicalNot, in[0])};
    case OP_BITWISE_NOT: return need(in, 1, code), std::vector<TensorP>{unary(k::kBitNot, in[0])};
    case OP_SCALAR_MUL: need(in, 1, code); return {unary(k::kScale, in[0], (float)fp(f, 0, code))};
    case OP_POW: need(in, 1, code); return {unary(k::kPow, in[0], (float)fp(f, 0, code))};
    case OP_CLAMP: need(in, 1, code); return {unary(k::kClamp, in[0], (float)fp(f, 0, code), (float)fp(f, 1, code))};
    case OP_SHL: need(in, 1, code); return {unary(k::kShl, in[0], (float)ip(iv, 0, code))};
    case OP_SHR: need(in, 1, code); return {unary(k::kShr, in[0], (float)ip(iv, 0, code))};
    case OP_CAST: need(in, 1, code); return {cast(in[0], dt_param(ip(iv, 0, code)))};
    case OP_QUANTIZE:
      need(in, 1, code);
      return {quantize(in[0], dt_param(ip(iv, 0, code)), (float)fp(f, 0, code), (int)ip(iv, 1, code))};
    case OP_DEQUANTIZE:
      need(in, 1, code);
      return {dequantize(in[0], dt_param(ip(iv, 0, code)), (float)fp(f, 0, code), (int)ip(iv, 1, code))};
    case OP_SOFTMAX: need(in, 1, code); return {softmax(in[0], k::kSoftmax)};
    case OP_LOG_SOFTMAX: need(in, 1, code); return {softmax(in[0], k::kLogSoftmax)};
    case OP_SOFTMAX_CAUSAL: need(in, 1, code); return {softmax(in[0], k::kSoftmaxCausal)};
    case OP_LAYER_NORM:
      need(in, 3, code);
      return {layer_norm(in[0], in[1], in[2], f.empty() ? 1e-5f : (float)f[0])};
    case OP_SUM: need(in, 1, code); return {row_reduce(k::kRSum, in[0])};
    case OP_MEAN: need(in, 1, code); return {row_reduce(k::kRMean, in[0])};
    case OP_AMAX: need(in, 1, code); return {row_reduce(k::kRAmax, in[0])};
    case OP_ARGMAX: need(in, 1, code); return {row_reduce(k::kRArgmax, in[0])};
    case OP_VAR: need(in, 1, code); return {row_reduce(k::kRVar, in[0], iv.empty() ? 1 : (int)iv[0])};
    case OP_STD: {
      need(in, 1, code);
      TensorP v = row_reduce(k::kRVar, in[0], iv.empty() ? 1 : (int)iv[0]);
      return {unary(k::kSqrt, v)};
    }
    case OP_SUM_DIM:
      need(in, 1, code);
      return {sum_dim(in[0], ip(iv, 0, code), iv.size() > 1 && iv[1] != 0)};
    case OP_MEAN_ALL: need(in, 1, code); return {mean_all(in[0])};
    case OP_MSE_LOSS: need(in, 2, code); return {mse_loss(in[0], in[1])};
    case OP_MSE_LOSS_BACKWARD: need(in, 3, code); return {mse_loss_backward(in[0], in[1], in[2])};
    case OP_SOFTMAX_BACKWARD: need(in, 2, code); return {softmax_backward(in[0], in[1])};
    case OP_LAYER_NORM_BACKWARD:
    case OP_LAYER_NORM_GRADS:
      // (grad_output, input, gamma[, saved mean, saved rstd]), eps (default
      // 1e-5, crates/python/src/lib.rs:1159)
      if (in.size() != 3 && in.size() != 5) fail("%s expects 3 or 5 tensor inputs", op_name(code));
      return layer_norm_grads(in[0], in[1], in[2], f.empty() ? 1e-5f : (float)f[0], code == OP_LAYER_NORM_GRADS,
                              in.size() == 5 ? in[3] : nullptr, in.size() == 5 ? in[4] : nullptr);
    case OP_GELU_BACKWARD:
    case OP_GELU_TANH_BACKWARD: need(in, 2, code); return {gelu_backward(in[0], in[1], false)};
    case OP_GELU_EXACT_BACKWARD: need(in, 2, code); return {gelu_backward(in[0], in[1], true)};
    case OP_EMBEDDING_BACKWARD: need(in, 2, code); return {embedding_backward(in[0], in[1], ip(iv, 0, code))};
    case OP_THRESHOLD_BACKWARD:
      need(in, 2, code);
      return {threshold_backward(in[0], in[1], f.empty() ? 0.f : (float)f[0])};
    case OP_EMBEDDING: need(in, 2, code); return {embedding(in[0], in[1])};
    case OP_INDEX_SELECT: need(in, 2, code); return {index_select(in[0], (int)ip(iv, 0, code), in[1])};
    case OP_GATHER: need(in, 2, code); return {gather(in[0], (int)ip(iv, 0, code), in[1])};
    case OP_CONCAT: need(in, 2, code); return {concat(in[0], in[1], (int)ip(iv, 0, code))};
    case OP_SLICE:
      need(in, 1, code);
      return {slice(in[0], (int)ip(iv, 0, code), ip(iv, 1, code), ip(iv, 2, code))};
    case OP_RESHAPE: need(in, 1, code); return {reshape(in[0], iv)};
    case OP_TRANSPOSE:
      need(in, 1, code);
      if (in[0]->ndim < 2) fail("transpose requires at least 2D tensor, got %s", shape_str(in[0]->dims()).c_str());
      return {transpose_dims(in[0], in[0]->ndim - 2, in[0]->ndim - 1)};
    case OP_TRANSPOSE_DIMS: {
      need(in, 1, code);
      int d0 = (int)ip(iv, 0, code), d1 = (int)ip(iv, 1, code);
      if (d0 == d1 && d0 >= 0 && d0 < in[0]->ndim) return {in[0]};
      return {transpose_dims(in[0], d0, d1)};
    }
    case OP_MATMUL: need(in, 2, code); return {matmul(in[0], in[1])};
    case OP_MATMUL_EX:
      need(in, 2, code);
      return {matmul(in[0], in[1], ip(iv, 0, code) != 0, ip(iv, 1, code) != 0)};
    case OP_LINEAR: {
      // y = act(x W^T + b), W in torch layout [out, in]
      if (in.size() != 2 && in.size() != 3) fail("linear expects 2 or 3 inputs");
      Epilogue e;
      if (in.size() == 3) e.bias = in[2];
      e.act = iv.empty() ? 0 : (int)iv[0];
      return {matmul(in[0], in[1], false, true, &e)};
    }
    case OP_ADD_BIAS: need(in, 2, code); return {add_bias(in[0], in[1])};
    case OP_ATTENTION:
    case OP_ATTENTION_CAUSAL:
      // optional f[0]: the softmax scale (default 1/sqrt(D))
      need(in, 3, code);
      return {attention(in[0], in[1], in[2], code == OP_ATTENTION_CAUSAL, false, f.empty() ? 0.f : (float)f[0])};
    case OP_WHERE: need(in, 3, code); return {where(in[0], in[1], in[2])};
    case OP_MASKED_FILL: need(in, 2, code); return {masked_fill(in[0], in[1], (float)fp(f, 0, code))};
    case OP_TRIU: need(in, 1, code); return {tri(in[0], true, iv.empty() ? 0 : iv[0])};
    case OP_TRIL: need(in, 1, code); return {tri(in[0], false, iv.empty() ? 0 : iv[0])};
    case OP_QUANTIZE_PER_ROW: {
      need(in, 1, code);
      auto qs = quantize_per_row(in[0]);
      return {qs.first, qs.second};
    }
    case OP_DEQUANTIZE_PER_ROW:
      need(in, 2, code);
      return {dequantize_per_row(in[0], in[1], iv.empty() ? DType::F32 : dt_param(iv[0]))};
    case OP_LINEAR_INT8: need(in, 3, code); return {linear_int8(in[0], in[1], in[2])};
    case OP_DECODE_ATTENTION:
      if (in.size() == 6) return {decode_attention(in[0], in[1], in[2], in[3], in[4], in[5])};
      need(in, 4, code);
      return {decode_attention(in[0], in[1], in[2], in[3])};
    case OP_PACK_WEIGHT: need(in, 1, code); return {pack_weight(in[0])};
    case OP_PACK_WEIGHT_X3: need(in, 1, code); return {pack_weight_x3(in[0])};
    case OP_MATMUL_PACKED: need(in, 2, code); return {matmul_packed(in[0], in[1], ip(iv, 0, code))};
    case OP_PACK_ROWS_X3: need(in, 1, code); return {pack_rows_x3(in[0])};
    case OP_MATMUL_PP: need(in, 2, code); return {matmul_pp(in[0], ip(iv, 0, code), in[1], ip(iv, 1, code))};
    case OP_ROW_STATS_X3: need(in, 1, code); return {row_stats_x3(in[0])};
    case OP_MATMUL_PP_NORM:
      need(in, 4, code);
      return {matmul_pp_norm(in[0], in[1], ip(iv, 0, code), in[2], in[3], ip(iv, 1, code),
                             f.empty() ? 1e-5f : (float)f[0])};
    case OP_SGD_MATMUL:
      // (w, a, b) or (w, a, b, bias): the bias step rides with the weight step
      if (in.size() != 4) need(in, 3, code);
      return {sgd_matmul_(in[0], in[1], in[2], iv.size() > 0 && iv[0], iv.size() > 1 && iv[1], (float)fp(f, 0, code),
                          in.size() == 4 ? in[3] : nullptr)};
    case OP_SGD_SUM_ROWS: need(in, 2, code); return {sgd_sum_rows_(in[0], in[1], (float)fp(f, 0, code))};
    case OP_LINEAR_MSE_BACKWARD_SGD: {
      // (h, w, b, y); iv[0]: also return the input gradient
      need(in, 4, code);
      auto r = linear_mse_backward_sgd_(in[0], in[1], in[2], in[3], (float)fp(f, 0, code), !iv.empty() && iv[0]);
      return {r.first, r.second};
    }
    case OP_MLP2_SGD_STEP:
      // (x, y, w1, b1, w2, b2)
      need(in, 6, code);
      return {mlp2_sgd_step_(in[0], in[1], in[2], in[3], in[4], in[5], (float)fp(f, 0, code))};
    case OP_LINEAR_RELU_MSE_BACKWARD_SGD: {
      // (a, wh, bh, w, b, y); iv[0]: also return the input gradient
      need(in, 6, code);
      auto r = linear_relu_mse_backward_sgd_(in[0], in[1], in[2], in[3], in[4], in[5], (float)fp(f, 0, code),
                                             !iv.empty() && iv[0]);
      return {std::get<0>(r), std::get<1>(r), std::get<2>(r)};
    }
    case OP_LINEAR_BACKWARD_SGD_PAIR:
      // (w1, b1, g, h, w0, b0, x)
      need(in, 7, code);
      return {linear_backward_sgd_pair_(in[0], in[1], in[2], in[3], in[4], in[5], in[6], (float)fp(f, 0, code))};
    case OP_LINEAR_BACKWARD_SGD:
      // (w, b, g, a) or (w, b, g, a, mask)
      if (in.size() != 5) need(in, 4, code);
      return {linear_backward_sgd_(in[0], in[1], in[2], in[3], in.size() == 5 ? in[4] : nullptr,
                                   (float)fp(f, 0, code))};
    case OP_QKV_ATTENTION:
      need(in, 3, code);
      return {qkv_attention(in[0], in[1], in[2], ip(iv, 0, code), iv.size() > 1 ? iv[1] != 0 : true,
                            iv.size() > 2 ? iv[2] : 1, iv.size() > 3 && iv[3] != 0)};
    case OP_MSE_LOSS_GRAD: {
      need(in, 2, code);
      auto lg = mse_loss_grad(in[0], in[1]);
      return {lg.first, lg.second};
    }
    case OP_CONTIGUOUS: {
      need(in, 1, code);
      TensorP c = contiguous(in[0]);
      if (c == in[0]) {
        // always hand back a distinct tensor object sharing the storage
        auto v = std::make_shared<Tensor>(*c);
        v->node = nullptr;
        v->ext_refs = 0;
        c = v;
      }
      return {c};
    }
    case OP_FULL: {
      if (!in.empty()) fail("full takes no tensor inputs");
      DType dt = dt_param(ip(iv, 0, code));
      std::vector<int64_t> dims(iv.begin() + 1, iv.end());
      return {full(dt, dims, f.empty() ? 0.f : (float)f[0])};
    }
  }
  fail("unknown op code %d", code);
}

// ── lazy recording ─────────────────────────────────────────────────────────
std::vector<TensorP> record_op(int code, const std::vector<TensorP>& in, const std::vector<double>& f,
                               const std::vector<int64_t>& iv) {
  if (code == OP_SGD_MATMUL || code == OP_SGD_SUM_ROWS || code == OP_LINEAR_BACKWARD_SGD ||
      code == OP_LINEAR_MSE_BACKWARD_SGD || code == OP_MLP2_SGD_STEP || code == OP_LINEAR_BACKWARD_SGD_PAIR ||
      code == OP_LINEAR_RELU_MSE_BACKWARD_SGD)
    fail("%s updates its first operand in place: eager only", op_name(code));
  std::vector<TensorP> metas;
  {
    MetaScope ms;
    metas = run_op(code, in, f, iv);
  }
  auto node = std::make_shared<Node>();
  node->code = code;
  node->in = in;
  node->f = f;
  node->iv = iv;
  std::vector<TensorP> outs;
  for (size_t i = 0; i < metas.size(); ++i) {
    auto t = make_meta(metas[i]->dtype, metas[i]->dims());
    if (metas.size() == 1) {
      t->node = node;
    } else {
      // Multi-output ops: output i is a selector node on a shared producer.
      auto sel = std::make_shared<Node>();
      sel->code = -1 - (int)i;  // selector
      sel->in = {};
      sel->f = {};
      sel->iv = {};
      t->node = sel;
    }
    outs.push_back(t);
  }
  if (metas.size() > 1) {
    // Producer is shared through a hidden tensor held by every selector.
    auto prod = make_meta(metas[0]->dtype, metas[0]->dims());
    prod->node = node;
    for (auto& t : outs) {
      t->node->in = {prod};
      node->selectors.push_back(t);
    }
  }
  return outs;
}

// ── eval ───────────────────────────────────────────────────────────────────
static GraphStats g_stats;
GraphStats graph_stats() {
  GraphStats s = g_stats;
  s.launcher_calls = launcher_calls();
  return s;
}

namespace {

struct Group {
  Tensor* mm = nullptr;   // matmul node (absorbed)
  TensorP a, b;           // matmul operands
  TensorP bias;
  int act = k::kActNone;
  TensorP residual;
  bool has_bias = false;
  TensorP ln_gamma, ln_beta;  // a = layer_norm(a) folded into the GEMM
  float ln_eps = 1e-5f;
  int64_t packed_n = 0;       // b is packed decode weights of this many columns
  int64_t a_rows = -1;        // a is packed x3 rows of this many rows (matmul_pp)
  TensorP norm_stats, norm_cs;  // folded layer_norm of a (matmul_pp_norm)
  float norm_eps = 1e-5f;
};

// An elementwise chain planned for one fused_chain launch.
struct ChainPlan {
  k::ChainProgram prog;
  std::vector<const TensorP*> leaves;  // entries of the chain nodes' input lists
  int len = 0;
};

// The kernel op code of a node a chain may hold (float unary or arithmetic
// binary ops, crates/core/src/graph.rs is_elementwise), or -1.
int chain_op(int code) {
  switch (code) {
    case OP_ADD: case OP_SUB: case OP_MUL: case OP_DIV: case OP_MIN: case OP_MAX: return code - OP_ADD;
    case OP_NEG: return k::kNeg;
    case OP_RELU: return k::kRelu;
    case OP_EXP: return k::kExp;
    case OP_LOG: return k::kLog;
    case OP_SQRT: return k::kSqrt;
    case OP_ABS: return k::kAbs;
    case OP_SIGN: return k::kSign;
    case OP_TANH: return k::kTanh;
    case OP_SIN: return k::kSin;
    case OP_COS: return k::kCos;
    case OP_SIGMOID: return k::kSigmoid;
    case OP_GELU: return k::kGelu;
    case OP_GELU_EXACT: return k::kGeluExact;
    case OP_SCALAR_MUL: return k::kScale;
    case OP_POW: return k::kPow;
    case OP_CLAMP: return k::kClamp;
  }
  return -1;
}

bool chain_binary(int code) { return code >= OP_ADD && code <= OP_MAX; }

// Appends node n as the program's next step; `cur` is the chain node n
// consumes (nullptr for the chain's first node, whose left input is the
// starting accumulator).
template <typename LeafOf>
void add_chain_step(k::ChainProgram& prog, const Node* n, const Tensor* cur, LeafOf&& leaf_of) {
  k::ChainStep& st = prog.step[prog.n_steps++];
  st.op = chain_op(n->code);
  if (chain_binary(n->code)) {
    const bool acc_left = cur == nullptr || n->in[0].get() == cur;
    st.acc_rhs = acc_left ? 0 : 1;
    st.leaf = leaf_of(acc_left ? n->in[1] : n->in[0]);
  } else {
    st.leaf = -1;
    st.p0 = n->f.size() > 0 ? (float)n->f[0] : 0.f;
    st.p1 = n->f.size() > 1 ? (float)n->f[1] : 0.f;
  }
}

bool is_single_internal_use(const TensorP& t, const std::unordered_map<Tensor*, int>& uses, int planner_refs = 0) {
  if (!t->pending() || t->ext_refs != 0) return false;
  auto it = uses.find(t.get());
  if (it == uses.end() || it->second != 1) return false;
  // holders: the consumer's node input + the eval order list (+ references
  // the fusion planner itself keeps)
  return t.use_count() == 2 + planner_refs;
}

void assign(const TensorP& dst, const TensorP& src) {
  if (src->dtype != dst->dtype || src->ndim != dst->ndim)
    fail("internal: lazy result %s/%s does not match the recorded %s/%s", shape_str(src->dims()).c_str(),
         dtype_name(src->dtype), shape_str(dst->dims()).c_str(), dtype_name(dst->dtype));
  for (int i = 0; i < src->ndim; ++i)
    if (src->shape[i] != dst->shape[i]) fail("internal: lazy result shape mismatch");
  if (dst->buf) {
    // *_out ops preallocated the destination: copy into it.
    TensorP d = std::make_shared<Tensor>(*dst);
    d->node = nullptr;
    d->ext_refs = 0;
    d->set_contiguous_strides();
    ops::copy_into(d, src);
    dst->node.reset();
    return;
  }
  dst->buf = src->buf;
  dst->offset = src->offset;
  for (int i = 0; i < src->ndim; ++i) dst->strides[i] = src->strides[i];
  dst->node.reset();
}

}  // namespace

void eval(const TensorP& root) { eval_all({root}); }

void eval_all(const std::vector<TensorP>& roots) {
  // Post-order walk over the roots' pending ancestors (iterative), so the
  // fusion plan below sees every root's subgraph at once.
  std::vector<TensorP> order;
  std::unordered_set<Tensor*> seen;
  std::vector<std::pair<TensorP, size_t>> stack;
  for (const TensorP& root : roots) {
    if (!root || !root->pending() || seen.count(root.get())) continue;
    stack.push_back({root, 0});
    seen.insert(root.get());
    while (!stack.empty()) {
      auto& top = stack.back();
      Node* n = top.first->node.get();
      if (top.second < n->in.size()) {
        TensorP c = n->in[top.second++];
        if (c->pending() && !seen.count(c.get())) {
          seen.insert(c.get());
          stack.push_back({c, 0});
        }
      } else {
        order.push_back(top.first);
        stack.pop_back();
      }
    }
  }
  if (order.empty()) return;
  g_stats.evals++;
  g_stats.nodes += order.size();

  // Uses inside this subgraph.
  std::unordered_map<Tensor*, int> uses;
  for (auto& t : order)
    for (auto& c : t->node->in)
      if (c->pending()) uses[c.get()]++;

  // GEMM epilogue fusion: matmul -> [add_bias (2-D)] -> [gelu|gelu_exact|relu] -> [add residual],
  // plus a layer_norm of the group's output computed by its split-K reduction.
  std::unordered_map<Tensor*, Group> groups;  // keyed by the group's current final node
  std::unordered_set<Tensor*> absorbed;
  std::unordered_map<Tensor*, TensorP> post_ln;  // group final node (or embedding sum) -> layer_norm reading it
  std::unordered_set<Tensor*> emb_adds;            // embedding + embedding nodes run as one kernel
  std::unordered_map<Tensor*, TensorP> pack_of;    // group final node or paired layer_norm -> pack_rows_x3 of it
  std::unordered_map<Tensor*, TensorP> stats_of;   // group final node -> row_stats_x3 of it
  std::unordered_map<Tensor*, TensorP> attn_pack;  // attention node -> pack_rows_x3 of its head-merged output
  for (auto& t : order) {
    Node* n = t->node.get();
    if (n->code == OP_ADD_BIAS && t->ndim == 2) {
      const TensorP& x = n->in[0];
      if (x->pending() &&
          (x->node->code == OP_MATMUL || x->node->code == OP_MATMUL_PACKED || x->node->code == OP_MATMUL_PP ||
           x->node->code == OP_MATMUL_PP_NORM) &&
          x->ndim == 2 && is_single_internal_use(x, uses) && n->in[1]->ndim == 1) {
        Group g;
        g.mm = x.get();
        if (x->node->code == OP_MATMUL_PACKED) g.packed_n = x->node->iv[0];
        if (x->node->code == OP_MATMUL_PP || x->node->code == OP_MATMUL_PP_NORM) {
          g.a_rows = x->node->iv[0];
          g.packed_n = x->node->iv[1];
        }
        if (x->node->code == OP_MATMUL_PP_NORM) {
          g.a = x->node->in[0];
          g.norm_stats = x->node->in[1];
          g.b = x->node->in[2];
          g.norm_cs = x->node->in[3];
          g.norm_eps = x->node->f.empty() ? 1e-5f : (float)x->node->f[0];
          g.bias = n->in[1];
          g.has_bias = true;
          absorbed.insert(x.get());
          groups[t.get()] = g;
          continue;
        }
        // layer_norm -> matmul: the GEMM normalises its A rows itself when
        // its kernel can (ops::matmul falls back to an explicit layer_norm)
        const TensorP& la = x->node->in[0];
        // (only 16-bit GEMMs of <= 16 rows can: the skinny kernel; otherwise
        // the layer_norm stays a node, which the producing GEMM's split-K
        // reduction may compute)
        // (a pairing in post_ln, made when the layer_norm was visited as the
        // reader of an earlier group, holds one more reference to it)
        int paired = 0;
        for (auto& kv : post_ln) paired += kv.second.get() == la.get();
        // (and fp32 GEMMs with hi/lo-packed weights whose plan reads whole
        // rows: the row-panel kernel normalises its A rows in its prologue)
        const bool x3_fold = x->node->code == OP_MATMUL_PACKED && ops::is_x3_packed(x->node->in[1]) &&
                             la->dtype == DType::F32 &&
                             k::gemm_x3_ln_ok(la->shape[0], x->node->iv[0], la->shape[1]);
        if (g.a_rows < 0 && la->pending() && la->node->code == OP_LAYER_NORM && la->ndim == 2 &&
            ((la->dtype != DType::F32 && la->shape[0] <= 16) || x3_fold) && is_single_internal_use(la, uses, paired)) {
          for (auto pit = post_ln.begin(); pit != post_ln.end(); ++pit)
            if (pit->second.get() == la.get()) {  // normalised in this GEMM's prologue instead
              post_ln.erase(pit);
              break;
            }
          g.ln_gamma = la->node->in[1];
          g.ln_beta = la->node->in[2];
          g.ln_eps = la->node->f.empty() ? 1e-5f : (float)la->node->f[0];
          absorbed.insert(la.get());
          g.a = la->node->in[0];
        } else {
          g.a = la;
        }
        g.b = x->node->in[1];
        g.bias = n->in[1];
        g.has_bias = true;
        absorbed.insert(x.get());
        groups[t.get()] = g;
      }
    } else if (n->code == OP_GELU || n->code == OP_GELU_EXACT || n->code == OP_RELU) {
      const TensorP& x = n->in[0];
      auto it = groups.find(x.get());
      if (it != groups.end() && it->second.act == k::kActNone && !it->second.residual &&
          is_single_internal_use(x, uses)) {
        Group g = it->second;
        g.act = n->code == OP_RELU ? k::kActRelu : n->code == OP_GELU ? k::kActGelu : k::kActGeluExact;
        groups.erase(it);
        absorbed.insert(x.get());
        groups[t.get()] = g;
      }
    } else if (n->code == OP_PACK_ROWS_X3) {
      // Packed rows written by their producer: a packed-weight GEMM group's
      // row-panel epilogue, or the split-K reduction (or fused embedding)
      // that computes the layer_norm being packed.  The fp32 matrix is then
      // never stored.
      const TensorP& x = n->in[0];
      if (!x->pending() || x->dtype != DType::F32 || x->ndim != 2 || x->shape[1] % 16 != 0) continue;
      // attention [H, T, D] -> transpose(0, 1) -> reshape [T, H*D] -> packed
      // rows: the attention kernel writes the packed rows itself
      if (x->node->code == OP_RESHAPE && is_single_internal_use(x, uses)) {
        const TensorP& y = x->node->in[0];
        if (y->pending() && y->node->code == OP_TRANSPOSE_DIMS && y->ndim == 3 && y->node->iv.size() == 2 &&
            std::min(y->node->iv[0], y->node->iv[1]) == 0 && std::max(y->node->iv[0], y->node->iv[1]) == 1 &&
            is_single_internal_use(y, uses)) {
          const TensorP& a = y->node->in[0];
          if (a->pending() && (a->node->code == OP_ATTENTION || a->node->code == OP_ATTENTION_CAUSAL) &&
              a->ndim == 3 && a->dtype == DType::F32 && x->shape[0] == a->shape[1] &&
              x->shape[1] == a->shape[0] * a->shape[2] && is_single_internal_use(a, uses)) {
            attn_pack[a.get()] = t;
            absorbed.insert(x.get());
            absorbed.insert(y.get());
            continue;
          }
        }
      }
      auto git = groups.find(x.get());
      if (git != groups.end() && git->second.packed_n > 0 && ops::is_x3_packed(git->second.b) &&
          !post_ln.count(x.get()) && !pack_of.count(x.get())) {
        pack_of[x.get()] = t;
        continue;
      }
      int paired = 0;
      for (auto& kv : post_ln) paired += kv.second.get() == x.get();
      if (paired == 1 && x->node->code == OP_LAYER_NORM && is_single_internal_use(x, uses, 1)) {
        pack_of[x.get()] = t;
        absorbed.insert(x.get());
      }
    } else if (n->code == OP_ROW_STATS_X3) {
      // row statistics from the producing packed-weight GEMM's epilogue
      const TensorP& x = n->in[0];
      auto git = groups.find(x.get());
      if (x->pending() && git != groups.end() && git->second.packed_n > 0 && ops::is_x3_packed(git->second.b) &&
          !post_ln.count(x.get()) && !stats_of.count(x.get()) && x->ndim == 2 && x->dtype == DType::F32)
        stats_of[x.get()] = t;
    } else if (n->code == OP_LAYER_NORM && t->ndim == 2) {
      const TensorP& x = n->in[0];
      // (computed where x is, which comes before gamma and beta in the walk:
      // they must already hold their values)
      if ((groups.count(x.get()) || emb_adds.count(x.get())) && !post_ln.count(x.get()) && n->in[1]->ndim == 1 &&
          n->in[2]->ndim == 1 && !n->in[1]->pending() && !n->in[2]->pending())
        post_ln[x.get()] = t;
    } else if (n->code == OP_ADD && n->in[0]->pending() && n->in[1]->pending() &&
               n->in[0]->node->code == OP_EMBEDDING && n->in[1]->node->code == OP_EMBEDDING &&
               n->in[0]->dims() == t->dims() && n->in[1]->dims() == t->dims() &&
               is_single_internal_use(n->in[0], uses) && is_single_internal_use(n->in[1], uses) &&
               ops::embedding_add_fusable(n->in[0]->node->in[0], n->in[0]->node->in[1], n->in[1]->node->in[0],
                                          n->in[1]->node->in[1])) {
      // token + position embedding: one launch (and the layer_norm reading
      // the sum, when one does, below)
      emb_adds.insert(t.get());
      absorbed.insert(n->in[0].get());
      absorbed.insert(n->in[1].get());
    } else if (n->code == OP_ADD) {
      for (int side = 0; side < 2; ++side) {
        const TensorP& x = n->in[side];
        const TensorP& other = n->in[1 - side];
        auto it = groups.find(x.get());
        if (it == groups.end() || it->second.residual || !is_single_internal_use(x, uses)) continue;
        // Only a same-shape, same-dtype add folds into the epilogue: the GEMM
        // writes its own output shape, so an add that broadcasts the GEMM
        // output (a [1, N] product plus an [M, N] residual, or a 2-D product
        // plus a 3-D one) stays a node of its own.
        if (other->dims() != t->dims() || x->dims() != t->dims() || other->dtype != x->dtype ||
            other.get() == x.get())
          continue;
        Group g = it->second;
        g.residual = other;
        groups.erase(it);
        absorbed.insert(x.get());
        groups[t.get()] = g;
        break;
      }
    }
  }

  // Group outputs whose packed rows or statistics come from their GEMM's
  // epilogue: stored in fp32 as well only when something else reads them
  // (another node, or a tensor held outside the graph).
  std::unordered_set<Tensor*> c_needed;
  for (auto& t : order) {
    Tensor* p = t.get();
    if (!groups.count(p)) continue;
    const int special = (pack_of.count(p) ? 1 : 0) + (stats_of.count(p) ? 1 : 0);
    if (!special) continue;
    auto u = uses.find(p);
    const int internal = u == uses.end() ? 0 : u->second;
    if (internal != special || t.use_count() != 1 + special) c_needed.insert(p);
  }

  // Elementwise chains (crates/core/src/fusion.rs:60-141, run on every eval
  // at lazy.rs:237): starting at an elementwise node, follow its single
  // consumer while that consumer is elementwise too and the current node
  // has no other user, inside or outside the graph.  A chain of two or more
  // runs as one fused_chain launch at its last node; the nodes before it are
  // absorbed.  Nodes the GEMM planning above claimed stay with their GEMM.
  std::unordered_map<Tensor*, ChainPlan> chains;  // keyed by the chain's last node
  {
    std::unordered_map<Tensor*, size_t> pos;
    for (size_t i = 0; i < order.size(); ++i) pos[order[i].get()] = i;
    std::unordered_map<Tensor*, Tensor*> consumer;  // valid for tensors with one internal use
    for (auto& t : order)
      for (auto& c : t->node->in)
        if (c->pending()) consumer[c.get()] = t.get();
    auto fusable = [&](Tensor* t) {
      return chain_op(t->node->code) >= 0 && (t->dtype == DType::F32 || t->dtype == DType::F16 ||
                                              t->dtype == DType::BF16) &&
             !absorbed.count(t) && !groups.count(t) && !emb_adds.count(t) && !post_ln.count(t);
    };
    std::unordered_set<Tensor*> taken;
    for (size_t i = 0; i < order.size(); ++i) {
      Tensor* s = order[i].get();
      if (taken.count(s) || !fusable(s)) continue;
      std::vector<Tensor*> nodes{s};
      std::vector<const TensorP*> leaves;
      k::ChainProgram prog;
      auto leaf_of = [&](const TensorP& x) {
        for (size_t j = 0; j < leaves.size(); ++j)
          if (leaves[j]->get() == x.get()) return (int)j;
        leaves.push_back(&x);
        return (int)leaves.size() - 1;
      };
      // first node: acc = its (left) input, then the node as a step
      const Node* n0 = s->node.get();
      prog.first = leaf_of(n0->in[0]);
      add_chain_step(prog, n0, nullptr, leaf_of);
      Tensor* cur = s;
      for (;;) {
        auto ci = consumer.find(cur);
        if (ci == consumer.end() || !is_single_internal_use(order[pos[cur]], uses)) break;
        Tensor* nx = ci->second;
        if (taken.count(nx) || !fusable(nx) || nx->dtype != s->dtype) break;
        const Node* nn = nx->node.get();
        // the other operand (if any) must fit in the leaf table
        int extra = 0;
        if (nn->in.size() == 2) {
          const TensorP& other = nn->in[0].get() == cur ? nn->in[1] : nn->in[0];
          bool known = false;
          for (auto* l : leaves) known |= l->get() == other.get();
          extra = known ? 0 : 1;
        }
        if (prog.n_steps >= k::kChainMaxSteps || (int)leaves.size() + extra > k::kChainMaxLeaves) break;
        add_chain_step(prog, nn, cur, leaf_of);
        nodes.push_back(nx);
        cur = nx;
      }
      if (nodes.size() < 2) continue;
      prog.n_leaves = (int)leaves.size();
      for (Tensor* t : nodes) taken.insert(t);
      for (size_t j = 0; j + 1 < nodes.size(); ++j) absorbed.insert(nodes[j]);
      ChainPlan cp;
      cp.prog = prog;
      cp.leaves = leaves;
      cp.len = (int)nodes.size();
      chains[cur] = cp;
    }
  }

  // Read-ahead of packed weights: a launch that leaves most CUs idle (a
  // split-K layer_norm reduction, the fused embedding, a row panel, the
  // decode attention) gets
  // extra blocks that read the packed weights of the GEMMs after it, up to
  // and including the next such launch, so that those GEMMs find their
  // weights in the Infinity Cache instead of HBM (GPT-2 small forward
  // 0.695 -> 0.681 ms with the reduction and embedding launches carrying).
  // Results are unchanged.
  std::vector<k::Prefetch> pf_for(order.size());
  {
    auto x3_weights = [&](size_t j) -> const Tensor* {
      auto it = groups.find(order[j].get());
      if (it == groups.end() || absorbed.count(order[j].get())) return nullptr;
      const Group& g = it->second;
      // packed weights of either layout: fp32 hi/lo (row panels) or 16-bit
      // decode-packed (skinny GEMMs)
      if (g.packed_n <= 0 || g.b->pending() || !g.b->buf) return nullptr;
      return g.b.get();
    };
    auto reads_ahead = [&](size_t j) {
      Tensor* t = order[j].get();
      if (absorbed.count(t)) return false;
      auto git = groups.find(t);
      if (git != groups.end()) {
        if (post_ln.count(t)) return true;
        // A packed-row panel with a layer_norm folded in, and a split panel
        // that finishes its tiles in its own launch, leave CUs idle too.
        // GPT-2 small forward 0.6124 -> 0.5885 ms with the folded panels
        // (c_attn, c_fc) carrying; the unfolded c_proj panel carrying as
        // well measured 0.598 ms, the attention launch carrying in place of
        // c_attn 0.613 ms.
        const Group& g = git->second;
        if (g.a_rows < 1 || g.packed_n <= 0 || !ops::is_x3_packed(g.b)) return false;
        if (g.norm_stats) return true;
        const int64_t K = g.b->shape[1] * 16;
        return k::gemm_x3_rows_out_ok(g.a_rows, g.packed_n, K, true) &&
               !k::gemm_x3_panel_ok(g.a_rows, g.packed_n, K, true);
      }
      // the whole-row decode attention runs 160 blocks for GPT-2 large's
      // 8 x 20 heads: it reads ahead the projection's weights (C4 decode
      // step 1.2746 -> 1.2660 and 1.3291 -> 1.3261 ms, alternating runs on
      // two boxes; reading c_fc's as well measured 1.2977, and the 80-block
      // projection and fc2 skinny launches as carriers 1.3793)
      if (t->node && t->node->code == OP_DECODE_ATTENTION) return true;
      return emb_adds.count(t) > 0;
    };
    for (size_t i = 0; i < order.size(); ++i) {
      if (!reads_ahead(i)) continue;
      k::Prefetch& pf = pf_for[i];
      int64_t total = 0;
      for (size_t j = i + 1; j < order.size() && pf.n < 3; ++j) {
        if (const Tensor* w = x3_weights(j)) {
          const int64_t nb = (int64_t)w->nbytes();
          if (pf.n > 0 && total + nb > (12LL << 20)) break;  // keep the reads inside the launch's latency
          pf.ptr[pf.n] = w->data();
          pf.bytes[pf.n] = nb;
          total += nb;
          ++pf.n;
        }
        if (reads_ahead(j)) break;
      }
    }
  }

  // The read-ahead ranges are raw pointers into this walk's weights: clear
  // them when the walk ends, also when an op throws part way, so that no
  // later launch reads ahead from memory that may have been freed since.
  struct PrefetchClear {
    ~PrefetchClear() { k::set_prefetch(k::Prefetch{}); }
  } clear_prefetch;
  for (size_t i = 0; i < order.size(); ++i) {
    TensorP t = order[i];
    // Absorbed into a fused GEMM, or already filled by its multi-output
    // producer earlier in this walk.
    if (absorbed.count(t.get()) || !t->pending()) {
      order[i].reset();
      continue;
    }
    k::set_prefetch(pf_for[i]);
    Node* n = t->node.get();
    auto git = groups.find(t.get());
    auto cit = chains.find(t.get());
    std::vector<TensorP> res;
    if (cit != chains.end()) {
      const ChainPlan& cp = cit->second;
      std::vector<TensorP> leaves;
      for (const TensorP* l : cp.leaves) leaves.push_back(*l);
      res = {ops::fused_chain(leaves, cp.prog, t->dtype, t->dims())};
      g_stats.fused_chains++;
      g_stats.chain_nodes += cp.len;
      g_stats.launches_saved += cp.len - 1;
    } else if (git != groups.end()) {
      const Group& g = git->second;
      ops::Epilogue e;
      e.bias = g.bias;
      e.act = g.act;
      e.residual = g.residual;
      e.ln_gamma = g.ln_gamma;
      e.ln_beta = g.ln_beta;
      e.ln_eps = g.ln_eps;
      auto pit = post_ln.find(t.get());
      TensorP lnt = pit != post_ln.end() && pit->second->pending() ? pit->second : nullptr;
      const bool x3 = g.packed_n > 0 && ops::is_x3_packed(g.b);
      auto packed_product = [&](ops::PostLn* pl, ops::PackOut* po) {
        return g.a_rows >= 0 ? ops::matmul_pp(g.a, g.a_rows, g.b, g.packed_n, &e, pl, po)
                             : ops::matmul_packed(g.a, g.b, g.packed_n, &e, pl, po);
      };
      e.norm_stats = g.norm_stats;
      e.norm_cs = g.norm_cs;
      e.norm_eps = g.norm_eps;
      auto pk = pack_of.find(t.get());
      auto st = stats_of.find(t.get());
      if ((pk != pack_of.end() || st != stats_of.end()) && x3 && !lnt) {
        // packed rows and/or row statistics of the output from the same
        // launch; the fp32 output too when anything else reads it
        ops::PackOut po;
        po.want_pk = pk != pack_of.end();
        po.want_stats = st != stats_of.end();
        po.want_c = c_needed.count(t.get()) > 0;
        TensorP out = packed_product(nullptr, &po);
        if (po.want_pk) assign(pk->second, po.pk);
        if (po.want_stats) assign(st->second, po.stats);
        g_stats.fused_gemm_epilogues++;
        g_stats.launches_saved += (g.has_bias ? 1 : 0) + (g.act ? 1 : 0) + (g.residual ? 1 : 0) +
                                  (po.want_pk ? 1 : 0) + (po.want_stats ? 1 : 0);
        if (!po.want_c) {
          order[i].reset();
          continue;
        }
        assign(t, out);
        order[i].reset();
        continue;
      }
      if (lnt && (g.packed_n == 0 || x3)) {
        ops::PostLn pl;
        pl.gamma = lnt->node->in[1];
        pl.beta = lnt->node->in[2];
        pl.eps = lnt->node->f.empty() ? 1e-5f : (float)lnt->node->f[0];
        auto lp = pack_of.find(lnt.get());
        if (lp != pack_of.end() && x3) {
          pl.want_y = false;
          pl.want_pk = true;
        }
        res = {g.packed_n > 0 ? packed_product(&pl, nullptr)
                              : ops::matmul(g.a, g.b, false, false, &e, nullptr, &pl)};
        if (pl.want_pk) {
          assign(lp->second, pl.ypk);
          g_stats.launches_saved++;
        } else {
          assign(lnt, pl.y);
        }
        g_stats.launches_saved++;
      } else {
        res = {g.packed_n > 0 ? packed_product(nullptr, nullptr) : ops::matmul(g.a, g.b, false, false, &e)};
      }
      g_stats.fused_gemm_epilogues++;
      g_stats.launches_saved += (g.has_bias ? 1 : 0) + (g.act ? 1 : 0) + (g.residual ? 1 : 0) + (g.ln_gamma ? 1 : 0);
    } else if (n->code < 0) {
      fail("internal: multi-output selector reached without its producer");
    } else if (op_outputs(n->code) > 1) {
      // producer of a multi-output op: run once and fill every live output
      res = run_op(n->code, n->in, n->f, n->iv);
      for (size_t j = 0; j < n->selectors.size(); ++j) {
        TensorP s = n->selectors[j].lock();
        if (!s || !s->pending()) continue;
        int idx = -1 - s->node->code;
        assign(s, res[idx]);
      }
      t->buf = res[0]->buf;
      t->offset = res[0]->offset;
      for (int d = 0; d < t->ndim; ++d) t->strides[d] = res[0]->strides[d];
      t->node.reset();
      order[i].reset();
      continue;
    } else if (emb_adds.count(t.get())) {
      const Node* e1 = n->in[0]->node.get();
      const Node* e2 = n->in[1]->node.get();
      auto pit = post_ln.find(t.get());
      TensorP lnt = pit != post_ln.end() && pit->second->pending() ? pit->second : nullptr;
      if (lnt && lnt->dtype == t->dtype && lnt->dims() == t->dims()) {
        ops::PostLn pl;
        pl.gamma = lnt->node->in[1];
        pl.beta = lnt->node->in[2];
        pl.eps = lnt->node->f.empty() ? 1e-5f : (float)lnt->node->f[0];
        auto lp = pack_of.find(lnt.get());
        if (lp != pack_of.end()) {
          pl.want_y = false;
          pl.want_pk = true;
        }
        res = {ops::embedding_add(e1->in[0], e1->in[1], e2->in[0], e2->in[1], &pl)};
        if (pl.want_pk) {
          assign(lp->second, pl.ypk);
          g_stats.launches_saved++;
        } else {
          assign(lnt, pl.y);
        }
        g_stats.launches_saved += 3;
      } else {
        res = {ops::embedding_add(e1->in[0], e1->in[1], e2->in[0], e2->in[1], nullptr)};
        g_stats.launches_saved += 2;
      }
    } else if (n->code == OP_ATTENTION || n->code == OP_ATTENTION_CAUSAL) {
      const float scale = n->f.empty() ? 0.f : (float)n->f[0];
      auto ap = attn_pack.find(t.get());
      if (ap != attn_pack.end()) {
        TensorP pk = ops::attention_rows_x3(n->in[0], n->in[1], n->in[2], n->code == OP_ATTENTION_CAUSAL, scale);
        if (pk) {
          assign(ap->second, pk);
          g_stats.launches_saved += 1;
          order[i].reset();
          continue;
        }
        // the kernel cannot write packed rows: the absorbed head merge and
        // the pack run as ops after the attention
        TensorP o = ops::attention(n->in[0], n->in[1], n->in[2], n->code == OP_ATTENTION_CAUSAL, true, scale);
        const Node* pn = ap->second->node.get();
        const TensorP& xr = pn->in[0];
        assign(ap->second, ops::pack_rows_x3(ops::reshape(ops::transpose_dims(o, 0, 1), xr->dims())));
        order[i].reset();
        continue;
      }
      // Head-interleaved output: a following transpose(0,1)+reshape is free.
      res = {ops::attention(n->in[0], n->in[1], n->in[2], n->code == OP_ATTENTION_CAUSAL, true, scale)};
    } else {
      res = run_op(n->code, n->in, n->f, n->iv);
    }
    assign(t, res[0]);
    order[i].reset();
  }
}

}  // namespace agpu
