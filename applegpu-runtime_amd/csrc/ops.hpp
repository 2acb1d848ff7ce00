// Host-side op layer: validates shapes and dtypes (the reference's rules),
// picks layouts, allocates outputs from the pool and enqueues kernels on the
// runtime stream.  Used by both the eager C ABI and the lazy graph executor.
#pragma once

#include <tuple>

#include "core.hpp"
#include "kernels.hpp"

namespace agpu {
namespace ops {

// Layout helpers
TensorP contiguous(const TensorP& t);               // t itself when already contiguous
k::ND nd_for(const Tensor& t, const std::vector<int64_t>& out_dims);  // broadcast strides
k::ND nd_shape(const std::vector<int64_t>& dims);
// View of t as [rows, cols] with unit column stride; false if not expressible.
bool as_rows(const Tensor& t, int64_t* rows, int64_t* ld);
// A view of base's storage read as `dt`, at a byte offset from base's data
// (bounds-checked against the allocation).
TensorP view_bytes(const TensorP& base, DType dt, const std::vector<int64_t>& shape,
                   const std::vector<int64_t>& strides, int64_t offset_bytes);
TensorP view(const TensorP& base, const std::vector<int64_t>& shape, const std::vector<int64_t>& strides,
             int64_t offset_elems);
TensorP reshape(const TensorP& t, const std::vector<int64_t>& shape);   // view when possible
TensorP transpose_dims(const TensorP& t, int d0, int d1);                // always a view
TensorP slice(const TensorP& t, int dim, int64_t start, int64_t end);    // always a view

// Elementwise
TensorP binary(int op, const TensorP& a, const TensorP& b, float p0 = 0.f);
TensorP unary(int op, const TensorP& x, float p0 = 0.f, float p1 = 0.f);
TensorP cast(const TensorP& x, DType dt);
TensorP quantize(const TensorP& x, DType dt, float scale, int zero_point);
TensorP dequantize(const TensorP& x, DType dt, float scale, int zero_point);
TensorP where(const TensorP& c, const TensorP& x, const TensorP& y);
TensorP masked_fill(const TensorP& x, const TensorP& mask, float value);
TensorP tri(const TensorP& x, bool upper, int64_t diag);
TensorP threshold_backward(const TensorP& grad, const TensorP& input, float thr);
TensorP add_bias(const TensorP& x, const TensorP& bias);
// One launch for a chain of float elementwise ops (k::fused_chain): leaves
// broadcast onto `dims`, all of dtype `dt`.
TensorP fused_chain(const std::vector<TensorP>& leaves, const k::ChainProgram& prog, DType dt,
                    const std::vector<int64_t>& dims);
TensorP full(DType dt, const std::vector<int64_t>& dims, float value);
void axpy_inplace(const TensorP& self, const TensorP& other, float alpha);  // self += alpha*other
void copy_into(const TensorP& dst, const TensorP& src);                      // dst (any strides) = src

// Rows
TensorP softmax(const TensorP& x, int mode /* k::RowOp */);
TensorP layer_norm(const TensorP& x, const TensorP& g, const TensorP& b, float eps);
TensorP row_reduce(int op /* k::RedOp */, const TensorP& x, int correction = 0);
TensorP softmax_backward(const TensorP& dy, const TensorP& y);
// layer_norm backward: {dx} or, with params, {dx, dgamma, dbeta}.
std::vector<TensorP> layer_norm_grads(const TensorP& dy, const TensorP& x, const TensorP& g, float eps, bool params,
                                      const TensorP& mean = nullptr, const TensorP& rstd = nullptr);
TensorP gelu_backward(const TensorP& grad, const TensorP& x, bool exact);
TensorP embedding_backward(const TensorP& grad, const TensorP& idx, int64_t num_weights);
std::pair<TensorP, TensorP> quantize_per_row(const TensorP& x);             // (int8 codes, f32 scales)
TensorP dequantize_per_row(const TensorP& q, const TensorP& scale, DType dt);

// Reductions
TensorP sum_dim(const TensorP& x, int64_t dim, bool keepdim, float scale = 1.f);
TensorP mean_all(const TensorP& x);
TensorP mse_loss(const TensorP& a, const TensorP& b);
TensorP mse_loss_backward(const TensorP& g, const TensorP& a, const TensorP& b);

// Indexing
TensorP embedding(const TensorP& w, const TensorP& idx);
TensorP index_select(const TensorP& x, int dim, const TensorP& idx);
TensorP gather(const TensorP& x, int dim, const TensorP& idx);
TensorP concat(const TensorP& a, const TensorP& b, int dim);

// GEMM.  Batch dims of A and B broadcast (the lazy path's rule); `ta`/`tb`
// swap the last two dims of an operand in place (matmul_ex).
struct Epilogue {
  TensorP bias;       // [N]
  int act = k::kActNone;
  TensorP residual;   // same shape as the output
  TensorP mask;       // same shape as the output: out = mask > 0 ? out : 0
  float alpha = 1.f;
  // A = layer_norm(a, ln_gamma, ln_beta, ln_eps) over its last dim, fused into
  // the GEMM's operand load when the skinny kernel runs the product (else an
  // explicit layer_norm first)
  TensorP ln_gamma, ln_beta;
  float ln_eps = 1e-5f;
  // packed-A products only: A = layer_norm(X) with gamma folded into the
  // weights and beta into the bias; norm_stats = row_stats_x3(X), norm_cs =
  // the folded weights' column sums (matmul_pp_norm)
  TensorP norm_stats, norm_cs;
  float norm_eps = 1e-5f;
  // fp32, 2-D products: a_rowsum_acc[m] += alpha * sum_k op(a)(m, k)
  TensorP a_rowsum_acc;
};
// Also y = layer_norm(out, gamma, beta, eps) over the last dim; computed by
// the GEMM's split-K reduction when its plan has one, else by layer_norm.
struct PostLn {
  TensorP gamma, beta;
  float eps = 1e-5f;
  TensorP y;  // result
  // y as packed x3 rows too (fp32 output, N % 16 == 0), or instead of y
  bool want_y = true, want_pk = false;
  TensorP ypk;
};
// Outputs of a packed-weight product beyond fp32 C (want_c): the same
// values as packed x3 rows (pk) for a following packed-A product, and their
// row statistics per 32-column tile (stats, as row_stats_x3) for a
// layer_norm folded into that product.  Written by the product's epilogue
// when its plan allows, else by their own launches.
struct PackOut {
  bool want_c = true;
  bool want_pk = true;
  bool want_stats = false;
  TensorP pk, stats;
};
// No-allocation mode: the caller's output (`into`) and a caller-held split-K
// workspace of `cap` bytes; any operand that would need a device copy, and
// any plan whose workspace exceeds `cap`, is rejected instead.
struct NoAlloc {
  void* ws = nullptr;
  size_t cap = 0;
};
TensorP matmul(const TensorP& a, const TensorP& b, bool ta = false, bool tb = false,
               const Epilogue* epi = nullptr, const TensorP& into = nullptr, PostLn* post_ln = nullptr,
               const NoAlloc* no_alloc = nullptr);
// w1[i1] + w2[i2] in one launch (token + position embedding), and with ln
// also ln->y = layer_norm of the sum; embedding_add_fusable says whether the
// operands fit the kernel.
bool embedding_add_fusable(const TensorP& w1, const TensorP& i1, const TensorP& w2, const TensorP& i2);
TensorP embedding_add(const TensorP& w1, const TensorP& i1, const TensorP& w2, const TensorP& i2, PostLn* ln);
// SGD steps fused with their gradients, in place:
//   w += alpha * op(a) op(b)   (the weight gradient GEMM; w contiguous 2-D),
//     and with bias also bias += alpha * (row sums of op(a)) (a Linear
//     layer's bias step: op(a) = g^T, so its row sums are sum(g, 0));
//     the outer-product plan folds that sum into its operand packing
//   bias += alpha * sum(g, 0)  (g contiguous [rows, N])
TensorP sgd_matmul_(const TensorP& w, const TensorP& a, const TensorP& b, bool ta, bool tb, float alpha,
                    const TensorP& bias = nullptr);
TensorP sgd_sum_rows_(const TensorP& bias, const TensorP& g, float alpha);
// A Linear layer's backward and SGD step (y = a w^T + b, upstream gradient
// g [R, out]): with mask, returns g_in = (g w) where mask > 0, else 0 (the
// gradient of the layer input through the previous ReLU, from w before its
// update); then w += alpha g^T a and b += alpha sum(g, 0).  Without mask,
// returns w.  A layer with one output (w [1, N], fp32, mask == a) runs as one
// launch (linear1_backward_sgd); otherwise matmul with the mask and
// sgd_matmul_ with the bias.
TensorP linear_backward_sgd_(const TensorP& w, const TensorP& b, const TensorP& g, const TensorP& a,
                             const TensorP& mask, float alpha);
// The last Linear layer of an MSE regression (no activation) through its
// SGD step: z = h w^T + b, loss = mean((z - y)^2), g = dloss/dz, then
// linear_backward_sgd_(w, b, g, h, grad_in ? h : none, alpha).  Returns
// {loss, g_in} (g_in: the gradient of h through the previous ReLU, from w
// before its update; w itself when grad_in is false).  A one-output layer
// (w [1, N], fp32) is two launches (linear1_forward_mse, then
// linear1_backward_sgd, which also forms the loss); otherwise linear,
// mse_loss_grad and linear_backward_sgd_.
std::pair<TensorP, TensorP> linear_mse_backward_sgd_(const TensorP& h, const TensorP& w, const TensorP& b,
                                                     const TensorP& y, float alpha, bool grad_in);
// The backward and SGD steps of two stacked Linear layers, the lower one
// first in the net (no input gradient): y = relu(x w0^T + b0) = h, then
// h w1^T + b1 with output gradient g.  g0 = (g w1) * (h > 0) from w1
// before its step; then w1 += alpha g^T h, b1 += alpha sum(g, 0),
// w0 += alpha g0^T x, b0 += alpha sum(g0, 0).  Returns w0.  When both
// updates take the outer-product plan they run as one pack launch and one
// GEMM launch (k::gemm_outer_pair); otherwise as two sgd_matmul_ calls.
TensorP linear_backward_sgd_pair_(const TensorP& w1, const TensorP& b1, const TensorP& g, const TensorP& h,
                                  const TensorP& w0, const TensorP& b0, const TensorP& x, float alpha);
// The last hidden layer and the one-output regression layer of an MLP
// through their forward, MSE loss, backward and the output layer's SGD
// step: h = relu(a wh^T + bh), then linear_mse_backward_sgd_(h, w, b, y,
// alpha, grad_in).  Returns {loss, g_in, h}.  For fp32 with one output the
// hidden GEMM leaves its split-K partial sums unreduced and the output
// layer's forward reduces them (bias, ReLU, h written) while it forms z:
// three launches (GEMM, forward, backward) where the layered form has four.
std::tuple<TensorP, TensorP, TensorP> linear_relu_mse_backward_sgd_(const TensorP& a, const TensorP& wh,
                                                                    const TensorP& bh, const TensorP& w,
                                                                    const TensorP& b, const TensorP& y, float alpha,
                                                                    bool grad_in);
// One SGD step of Linear(w1, b1) -> ReLU -> Linear(w2, b2) with MSE loss
// against y, in place (w += alpha * grad, every gradient from the step's
// starting parameters); returns the loss [1].  Small fp32 shapes run as one
// launch (k::mlp2_step_ok), others as the layer ops above.
TensorP mlp2_sgd_step_(const TensorP& x, const TensorP& y, const TensorP& w1, const TensorP& b1, const TensorP& w2,
                       const TensorP& b2, float alpha);
// MSE loss and its gradient (upstream gradient 1): {loss [1], grad like a}.
std::pair<TensorP, TensorP> mse_loss_grad(const TensorP& a, const TensorP& b);
// Decode-step weights: wt [out N, in K] (fp16/bf16) rearranged for the skinny
// GEMM (the operands of one wave instruction contiguous), and x [M <= 16, K]
// times it: out [M, N] = epilogue(x @ wt^T).
TensorP pack_weight(const TensorP& wt);
// fp32 weights for few-row activations: b is the B operand [K, N] of x @ b
// (any strides), split into bf16 hi/lo and rearranged as MFMA fragments
// (k::pack_weights_x3): a BF16 tensor [N/32, K/16, 2, 64, 8].
TensorP pack_weight_x3(const TensorP& b);
bool is_x3_packed(const TensorP& t);
// x times packed weights: the 16-bit decode layout (pack_weight, at most 16
// rows) or the fp32 hi/lo layout (pack_weight_x3, any rows), with the
// epilogue and, for the fp32 layout, layer_norm of the output computed in the
// split-K reduction.
TensorP matmul_packed(const TensorP& x, const TensorP& packed, int64_t N, const Epilogue* epi = nullptr,
                      PostLn* post_ln = nullptr, PackOut* po = nullptr);
// Packed x3 rows of an fp32 matrix x [M, K] (K % 16 == 0): hi/lo bf16 in the
// MFMA A-operand order (k::pack_rows_x3), a BF16 tensor [ceil(M/32), K/16, 2,
// 64, 8].  The row count is not recoverable from the shape; matmul_pp takes it.
TensorP pack_rows_x3(const TensorP& x);
// apk (pack_rows_x3 of an [M, K] matrix) times fp32 weights packed by
// pack_weight_x3 ([K, N]): out [M, N] fp32 with the epilogue, and optionally
// layer_norm of the output (split-K reduction) and packed outputs.  Returns
// null when po asks for the packed output only.
TensorP matmul_pp(const TensorP& apk, int64_t M, const TensorP& packed, int64_t N, const Epilogue* epi = nullptr,
                  PostLn* post_ln = nullptr, PackOut* po = nullptr);
// Row statistics of an fp32 matrix x [M, N] (N % 32 == 0) per 32-column
// tile: [M, N/32, 2] = (sum, sum of squared deviations from the tile mean).
TensorP row_stats_x3(const TensorP& x);
// layer_norm(X) @ W + b as one packed product, for X given as packed rows
// (apk = pack_rows_x3(X)) with its statistics (stats = row_stats_x3(X)):
// folded = gamma[:, None] * W packed by pack_weight_x3, cs = column sums of
// gamma[:, None] * W, and the caller adds beta @ W + b as the bias.  The
// result is inv * (X @ folded - mean * cs) per row, with mean and
// inv = 1 / sqrt(var + eps) merged from the tile statistics.
TensorP matmul_pp_norm(const TensorP& apk, const TensorP& stats, int64_t M, const TensorP& folded,
                       const TensorP& cs, int64_t N, float eps, const Epilogue* epi = nullptr, PackOut* po = nullptr);
// int8 weights with per-row scales (out = x @ (q * scale[:,None])^T)
TensorP linear_int8(const TensorP& x, const TensorP& q, const TensorP& scale);

// GPT-2's attention block input side in one op: qkv = x w + b (x [B*T, K],
// w [K, 3d] row-major, b [3d]), split into n_head heads of Q, K, V, then
// (causal) attention; returns the head-merged output [B*T, d].  By default
// the projection (with its split-K reduction) and the attention run one after
// another.  read_partials (fp32, split-K plan): the attention kernel reads
// the projection's partial sums plus the bias instead, one launch fewer; at
// GPT-2 small's 128 tokens that measured slower (each head's K/V partials
// are re-read by all 8 of its query blocks).  Same values either way.
TensorP qkv_attention(const TensorP& x, const TensorP& w, const TensorP& b, int64_t n_head, bool causal,
                      int64_t batch, bool read_partials = false);
// Attention over [..., T, D] operands (leading dims shared by q, k, v).
// out_layout_thd: store the output physically as [..., T, H, D] (the result
// is still logically [..., H, T, D]) so a following head merge is free.
// scale: the softmax scale; 0 means 1/sqrt(D), the reference's
// (crates/core/src/ops.rs:1531-1620).
TensorP attention(const TensorP& q, const TensorP& k, const TensorP& v, bool causal,
                  bool out_layout_thd = false, float scale = 0.f);
// The same attention (fp32, fused kernel) with its output written as packed
// x3 rows (pack_rows_x3) of the [B*Tq, H*D] matrix of head-merged query rows:
// the A operand of the following projection (matmul_pp), never stored in
// fp32.  Null when the fused fp32 kernel cannot take the operands.
TensorP attention_rows_x3(const TensorP& q, const TensorP& k, const TensorP& v, bool causal, float scale = 0.f);
// q [B, H, Tq, D] against the first lens[b] rows of the [B, H, Tmax, D] caches
// (lens int32 [B] on the device; the queries' own keys are the last Tq of
// them); the output is logically [B, H, Tq, D], stored as [B, Tq, H, D].
// With k_new / v_new ([B, H, 1, D], Tq == 1) the step's own K and V rows are
// appended by the same launch: they become cache row lens[b] - 1 (dropped
// when lens[b] exceeds the cache), so the caches are updated in place.
TensorP decode_attention(const TensorP& q, const TensorP& k_cache, const TensorP& v_cache, const TensorP& lens,
                         const TensorP& k_new = nullptr, const TensorP& v_new = nullptr);
// cache[b, h, pos[b] + t, :] = rows[b, h, t, :] (pos int32 [B] on the device);
// an optional second cache/rows pair of the same shape in the same launch.
void kv_write(const TensorP& cache, const TensorP& rows, const TensorP& pos, const TensorP& cache2 = nullptr,
              const TensorP& rows2 = nullptr);

}  // namespace ops
}  // namespace agpu
