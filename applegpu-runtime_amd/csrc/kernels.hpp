// Launchers for the gfx950 kernels.  Every launcher enqueues on the stream it
// is given and returns immediately; shapes are checked by the caller (ops.cpp)
// before anything is launched.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "core.hpp"

namespace agpu {
namespace k {

// N-D strided operand for elementwise kernels (element strides; 0 = broadcast).
struct ND {
  int ndim = 0;
  int64_t shape[kMaxDims] = {};
  int64_t stride[kMaxDims] = {};
};

// ── elementwise ───────────────────────────────────────────────────────────
enum Bin : int {
  kAdd, kSub, kMul, kDiv, kMin, kMax, kMod, kAnd, kOr, kXor,
  kLt, kGt, kLe, kGe, kEq, kNe,
  kThresholdBwd,  // out = b > p0 ? a : 0   (a = grad, b = input)
  kSoftmaxBwd,    // unused by the binary launcher (row kernel)
  kGeluBwd,       // out = a * gelu_tanh'(b)  (a = grad, b = input)
  kGeluExactBwd,  // out = a * gelu_erf'(b)
};
enum Un : int {
  kNeg, kRelu, kExp, kLog, kSqrt, kAbs, kSign, kTanh, kSin, kCos, kSigmoid,
  kGelu, kGeluExact, kScale, kPow, kClamp, kBitNot, kLogicalNot, kShl, kShr,
  kCopy,          // also used for dtype casts (in != out dtype)
  kQuantize,      // round-half-away(x / p0) + p1, clamped to the int8/uint8 range
  kDequantize,    // (q - p1) * p0
  kFill,          // out = p0
};

// out has contiguous shape `so`; a/b are read through their own strides.
void binary(int op, DType in, DType out, const void* a, const ND& sa, const void* b,
            const ND& sb, void* o, const ND& so, float p0, hipStream_t s);
void unary(int op, DType in, DType out, const void* x, const ND& sx, void* o, const ND& so,
           float p0, float p1, hipStream_t s);
void where(DType cdt, DType dt, const void* c, const ND& sc, const void* x, const ND& sx,
           const void* y, const ND& sy, void* o, const ND& so, hipStream_t s);
// out = in, with rows/cols above (triu) or below (tril) `diag` zeroed, over
// the last two dims of a contiguous tensor.
void tri(DType dt, bool upper, int64_t diag, const void* x, void* o, int64_t batch, int64_t rows,
         int64_t cols, hipStream_t s);
// y[i] += alpha * x[i], x broadcast through `sx` onto the contiguous shape `sy`.
void axpy(DType dt, void* y, const ND& sy, const void* x, const ND& sx, float alpha, hipStream_t s);
// out[i] = in[i] + bias[(i / channel_stride) % channels]
// (crates/core/src/kernel_templates.rs:747-762)
void add_bias(DType dt, const void* in, const void* bias, void* out, int64_t numel,
              int64_t channels, int64_t channel_stride, hipStream_t s);

// ── fused elementwise chains ──────────────────────────────────────────────
// One launch for a chain of float elementwise ops, the lazy executor's
// fusion of single-consumer chains (crates/core/src/fusion.rs:60-282).  The
// program is interpreted per element from the kernel arguments (no runtime
// compilation): acc = leaf[first]; then each step is acc = un(acc),
// acc = acc op leaf[j] or acc = leaf[j] op acc.  After every step acc is
// rounded to the chain's dtype, as the unfused node would have stored it, so
// results equal the op-by-op launches bit for bit.
constexpr int kChainMaxLeaves = 8;
constexpr int kChainMaxSteps = 16;
struct ChainStep {
  int32_t op = 0;       // Un code (unary step) or Bin code (binary step)
  int32_t leaf = -1;    // binary: the other operand's leaf index; unary: -1
  int32_t acc_rhs = 0;  // binary: the accumulator is the right operand
  float p0 = 0.f, p1 = 0.f;
};
struct ChainProgram {
  int32_t n_steps = 0, first = 0, n_leaves = 0;
  ChainStep step[kChainMaxSteps];
};
struct ChainLeaves {
  const void* ptr[kChainMaxLeaves] = {};
  ND nd[kChainMaxLeaves];             // strides over the output shape (0 = broadcast)
  int64_t period[kChainMaxLeaves] = {};  // filled by the launcher
};
// out (contiguous, shape `so`) = the program over the leaves; dt is F32, F16
// or BF16 for every leaf and the output.
void fused_chain(DType dt, const ChainProgram& prog, ChainLeaves leaves, void* out, const ND& so, hipStream_t s);

// ── row kernels (last dim, row stride `ld`, unit column stride) ───────────
enum RowOp : int { kSoftmax, kLogSoftmax, kSoftmaxCausal };
void softmax_rows(int op, DType dt, const void* x, int64_t ldx, void* y, int64_t ldy,
                  int64_t rows, int64_t cols, int64_t causal_rows, hipStream_t s);
void layer_norm(DType dt, const void* x, int64_t ldx, const void* gamma, const void* beta,
                void* y, int64_t rows, int64_t cols, float eps, hipStream_t s);
enum RedOp : int { kRSum, kRMean, kRAmax, kRArgmax, kRVar };
void row_reduce(int op, DType in, DType out, const void* x, int64_t ldx, void* y, int64_t rows,
                int64_t cols, int correction, hipStream_t s);
// layer_norm backward over contiguous [rows, cols] dy and x: dx with the
// statistics recomputed from x, or taken from mean_in/rstd_in ([rows], the
// input dtype) when given; stats (nullable) gets [rows][2] = (mean,
// 1/sqrt(var + eps)).  layer_norm_param_grads then forms dgamma and dbeta
// (column sums, fixed order) from dy, x and stats; `ws` holds
// layer_norm_param_ws_bytes(rows, cols).
void layer_norm_backward(DType dt, const void* dy, const void* x, const void* gamma, void* dx, float* stats,
                         const void* mean_in, const void* rstd_in, int64_t rows, int64_t cols, float eps,
                         hipStream_t s);
size_t layer_norm_param_ws_bytes(int64_t rows, int64_t cols);
void layer_norm_param_grads(DType dt, const void* dy, const void* x, const float* stats, void* dgamma, void* dbeta,
                            float* ws, int64_t rows, int64_t cols, hipStream_t s);
// x[r] = w1[i1[r]] + w2[i2[r]] over [rows, cols] (cols <= 2048; contiguous
// [vocab, cols] tables), and when gamma is given also y = layer_norm(x),
// into y and/or (fp32, cols % 16 == 0) ypk as packed x3 rows.
bool embedding_add_ok(int64_t cols);
void embedding_add(DType dt, const void* w1, DType i1_dt, const void* i1, int64_t v1, const void* w2, DType i2_dt,
                   const void* i2, int64_t v2, void* x, const void* gamma, const void* beta, void* y, void* ypk,
                   int64_t rows, int64_t cols, float eps, hipStream_t s);
// Softmax backward: dx = y * (dy - sum(dy * y)) per row.
void softmax_backward(DType dt, const void* dy, const void* y, void* dx, int64_t rows,
                      int64_t cols, hipStream_t s);
// Symmetric per-row int8: scale[r] = absmax(row)/127, q = clamp(rint(x/scale)).
void quantize_rows(DType in, const void* x, int8_t* q, float* scale, int64_t rows,
                   int64_t cols, hipStream_t s);
void dequantize_rows(DType out, const int8_t* q, const float* scale, void* y, int64_t rows,
                     int64_t cols, hipStream_t s);

// ── reductions ────────────────────────────────────────────────────────────
// Contiguous x viewed as [outer, red, inner] -> y[outer, inner] = scale * sum.
void sum_dim(DType dt, const void* x, void* y, int64_t outer, int64_t red, int64_t inner,
             float scale, hipStream_t s);
// Whole-tensor reductions into one element of dtype `dt` (`ws` >= 4 KB of
// scratch): kind 0 = scale * sum(x), kind 1 = scale * sum((a-b)^2).
size_t reduce_all_ws_bytes();
void reduce_all(int kind, DType dt, const void* a, const void* b, int64_t n, float scale,
                void* out, void* ws, hipStream_t s);
// MSE backward: dx = (a - b) * (2/n) * g[0]   (g: one element of dtype dt)
void mse_backward(DType dt, const void* a, const void* b, const void* g, void* dx, int64_t n,
                  hipStream_t s);
// y[c] += alpha * sum_r x[r, c] over a contiguous [rows, cols] x (SGD bias step).
void sum_rows_axpy(DType dt, const void* x, void* y, int64_t rows, int64_t cols, float alpha, hipStream_t s);
// MSE loss and gradient (upstream gradient 1) in one launch, n <= 65536.
bool mse_fused_ok(int64_t n);
void mse_loss_grad(DType dt, const void* a, const void* b, void* loss, void* grad, int64_t n, hipStream_t s);

// ── indexing ──────────────────────────────────────────────────────────────
void embedding(DType dt, const void* w, int64_t vocab, int64_t dim, DType idx_dt,
               const void* idx, int64_t n, void* out, hipStream_t s);
// dw [nw, dim] = per-row sums of the dy [n, dim] rows each index names, in
// token order (zeros elsewhere; indices outside [0, nw) add nothing).
void embedding_backward(DType dt, const void* dy, DType idx_dt, const void* idx, int64_t n, int64_t dim,
                        int64_t nw, void* dw, hipStream_t s);
// Gathers along `dim` of a contiguous [outer, size, inner] tensor.
// index_select: out[o, j, i] = x[o, idx[j], i]            (idx 1-D, length m)
// gather:       out[o, j, i] = x[o, idx[o, j, i], i]      (idx shaped like out)
void index_select(DType dt, const void* x, int64_t outer, int64_t size, int64_t inner,
                  DType idx_dt, const void* idx, int64_t m, void* out, hipStream_t s);
void gather(DType dt, const void* x, int64_t outer, int64_t size, int64_t inner, DType idx_dt,
            const void* idx, int64_t m, void* out, hipStream_t s);

// ── GEMM (MFMA) ───────────────────────────────────────────────────────────
enum Act : int { kActNone = 0, kActRelu = 1, kActGelu = 2, kActGeluExact = 3 };
struct Gemm {
  DType dt = DType::F32;      // A, B, C, bias and residual share this dtype
  int64_t M = 0, N = 0, K = 0, batch = 1;
  const void* A = nullptr; int64_t a_sm = 0, a_sk = 0, a_sb = 0;   // A(m,k)
  const void* B = nullptr; int64_t b_sk = 0, b_sn = 0, b_sb = 0;   // B(k,n)
  void* C = nullptr; int64_t c_sm = 0, c_sb = 0;                    // C(m,n), unit n stride
  // epilogue: v = alpha*acc (+ bias[n]) -> act -> (+ residual(m,n)) -> (mask(m,n) > 0 ? v : 0)
  float alpha = 1.f;
  const void* bias = nullptr;
  int act = kActNone;
  const void* residual = nullptr; int64_t r_sm = 0, r_sb = 0;
  const void* mask = nullptr; int64_t k_sm = 0, k_sb = 0;
  // int8 B with per-n fp32 scales (dequant fused into the operand load)
  const float* b_scale = nullptr;
  DType b_dt = DType::F32;
  // A rows layer-normalised on load (gamma, beta [K] of dtype dt; skinny
  // kernel only, see gemm_skinny_ln_ok)
  const void* ln_gamma = nullptr;
  const void* ln_beta = nullptr;
  float ln_eps = 1e-5f;
  // B in the skinny kernel's packed layout (pack_weights), 16-bit, M <= 16
  bool b_packed = false;
  // fp32 B split ahead of time into bf16 hi/lo MFMA fragments
  // (pack_weights_x3); A fp32 with unit k stride, K % 16 == 0, one batch
  bool b_x3 = false;
  // with b_x3: A given as packed x3 rows ([ceil(M/32), K/16, 2, 64, 8] bf16,
  // x3_row_offset in the kernels) instead of fp32; a_sm/a_sk unused
  bool a_x3 = false;
  // with b_x3: C also (or, with C null, only) written as packed x3 rows, for
  // a following packed-A GEMM (row-panel plans, N % 16 == 0)
  void* c_pk = nullptr;
  // split-K launches leave the partial sums in the workspace (the caller
  // consumes them) instead of reducing them into C
  bool no_reduce = false;
  // fp32 A only: acc[m] += alpha * sum_k A(m, k) (an SGD bias step beside a
  // weight-gradient product), computed by the outer-product plan's operand
  // packing; other plans leave it to the caller (gemm_a_rowsum_fused)
  void* a_rowsum_acc = nullptr;
  // Y = layer_norm(C) over N (gamma, beta [N]) computed by the split-K
  // reduction while it writes C (gemm_post_ln_fused); Y is [M, N] contiguous
  const void* pln_gamma = nullptr;
  const void* pln_beta = nullptr;
  void* pln_y = nullptr;
  float pln_eps = 1e-5f;
  // Y also (or, with pln_y null, only) written as packed x3 rows (N % 16 == 0)
  void* pln_ypk = nullptr;
  // with b_x3, unsplit row-panel plans: rs_out receives the output's row
  // statistics per 32-column tile ([M, N/32, 2]: sum, squared deviations
  // from the tile mean; N % 32 == 0); with rs_in (A's statistics [M,
  // rs_tiles, 2] over rs_n columns, packed A) the epilogue computes
  // inv * (acc - mean * rs_cs[n]) before the bias: a layer_norm of A whose
  // gamma is folded into the weights (rs_cs = column sums of the folded
  // weights) and whose beta is folded into the bias
  float* rs_out = nullptr;
  const float* rs_in = nullptr;
  const float* rs_cs = nullptr;
  int rs_tiles = 0;
  int64_t rs_n = 0;
  float rs_eps = 1e-5f;
  // the most workspace the caller can provide: a plan that would need more
  // (the outer-product plan's packed operands) is not taken
  size_t max_ws = SIZE_MAX;
};
// fp32 weights packed for the bf16x3 MFMA GEMM of few-row activations
// (gemm_x3p.hip): B(k, n) read through strides (b_sk, b_sn) is split into
// bf16 hi/lo and stored in the B-operand order of v_mfma_f32_32x32x16_bf16,
// zero-padded to whole 32-column strips and 16-deep k steps
// (packed_x3_elems bf16 elements).
int64_t packed_x3_elems(int64_t K, int64_t N);
void pack_weights_x3(const void* b, int64_t b_sk, int64_t b_sn, int64_t K, int64_t N, void* out, hipStream_t s);
// Launch plan of the packed-weight GEMM: 128-row tiles, 64 (wide) or 32
// columns, kt 16-deep k steps per block and K split `splits` ways.
// rows: one 32 x 32 block per output tile over the whole K, no split: with
// fp32 A, K = 64 kpw (kpw 4, 8, 12 or 16) and an optional layer_norm of A in
// the prologue; with packed A (apk), K = 128 kpw (kpw 2..12, even).
// split: a plan that ends in a split-K reduction is required (the reduction
// computes a layer_norm of the output).
// stream: packed A, many columns (a vocabulary head): one block per 128 rows
// x 128 columns over the whole K, so that every weight byte is read once.
struct X3Plan {
  bool rows = false;
  bool stream = false;
  bool apk = false;
  int kpw = 0;
  bool wide = true;
  int64_t tiles_m = 0, tiles_n = 0;
  int kt = 1, splits = 1;
};
X3Plan x3_plan(int64_t M, int64_t N, int64_t K, int cus, bool apk = false, bool split = false);
// Read-ahead of the next GEMMs' weights: the ranges set here are read by
// extra blocks of the next launch that supports it (the split-K layer_norm
// reductions, fp32 fused attention, the fused embedding), which then clears
// them; any other launch leaves them set.  Up to three ranges.
struct Prefetch {
  const void* ptr[3] = {nullptr, nullptr, nullptr};
  int64_t bytes[3] = {0, 0, 0};
  int n = 0;
};
void set_prefetch(const Prefetch& pf);
Prefetch take_prefetch();
// Row statistics per 32-column tile of an fp32 matrix [M, N] (N % 32 == 0,
// 16-byte aligned rows): out [M, N/32, 2] = (sum, sum of squared deviations
// from the tile mean), identical to what a row-panel GEMM writes (rs_out).
void row_tile_stats(const float* x, int64_t x_sm, int64_t M, int64_t N, float* out, hipStream_t s);
// Whether the packed-weight GEMM of this shape runs an unsplit row-panel
// plan (packed outputs and row statistics come from its epilogue).
bool gemm_x3_panel_ok(int64_t M, int64_t N, int64_t K, bool apk);
// Whether its plan is a row panel whose epilogue writes the output (and its
// packed rows and row statistics) in the same launch: unsplit, or split
// with every tile finished in the kernel by its last-arriving split.
bool gemm_x3_rows_out_ok(int64_t M, int64_t N, int64_t K, bool apk);
// Device address of the split row-panel tiles' arrival counters (looked up
// once at init on the runtime's device; false with the error set on failure).
bool split_counters_setup(std::string* err);
// Packed x3 rows of an fp32 matrix X [M, K] read through strides (x_sm,
// x_sk), K % 16 == 0: the A-operand counterpart of pack_weights_x3
// (packed_x3_elems(K, M) bf16 elements).
void pack_rows_x3(const void* x, int64_t x_sm, int64_t x_sk, int64_t M, int64_t K, void* out, hipStream_t s);
// Whether the packed-weight GEMM of this shape normalises its A rows in its
// prologue (the row-panel plan).
bool gemm_x3_ln_ok(int64_t M, int64_t N, int64_t K);
// Whether a packed-weight GEMM can take this A operand and problem.
bool gemm_x3_ok(const Gemm& g);
// Whether a packed-A, packed-weight GEMM of this shape can write its output
// as packed x3 rows (the packed-A row-panel plan).
bool gemm_x3_pk_out_ok(int64_t M, int64_t N, int64_t K);
// Whether the launch ends in a split-K reduction that can also produce
// layer_norm(C) (one batch, N <= 2048); otherwise the caller runs layer_norm.
bool gemm_post_ln_fused(const Gemm& g);
// Backward and SGD step of a Linear layer with one output, one launch:
// gin[r, j] = h[r, j] > 0 ? dz[r] * w[j] : 0 (gin may be null), then
// w[j] += alpha * sum_r dz[r] h[r, j] and (b non-null) b[0] += alpha *
// sum_r dz[r].  h [R, N] with row stride h_sm and unit column stride, dz
// [R] with stride dz_s, w [N] and gin [R, N] contiguous.
struct Lin1Bwd {
  const void* h; int64_t h_sm;
  const void* dz; int64_t dz_s;
  void* w; void* b; void* gin;
  int64_t R, N;
  float alpha;
  // optional (loss non-null): loss[0] = inv_n * sum_r (z[r] - y[r])^2, the
  // MSE of the layer's forward output z against y (contiguous [R]), by
  // block 0 before it updates b
  const void* z; const void* y; void* loss; float inv_n;
};
void linear1_backward_sgd(DType dt, const Lin1Bwd& a, hipStream_t s);
// Forward of a Linear layer with one output and the MSE gradient, one
// launch (one block per row): z[r] = h[r, :] . w + b[0], dz[r] = (z[r] -
// y[r]) * two_over_n.  h [R, N] with row stride h_sm and unit column
// stride; w [N], b [1], y, z and dz [R] contiguous.
// One SGD step of Linear(N0 -> N1) -> ReLU -> Linear(N1 -> N2) with MSE
// loss over all R x N2 outputs, in one workgroup (mlp_step.hip): x [R, N0],
// y [R, N2], W1 [N1, N0], b1 [N1], W2 [N2, N1], b2 [N2] contiguous fp32, the
// parameters updated in place (w += alpha * grad), loss [1] written.
struct Mlp2Step {
  const float* x; const float* y;
  float* w1; float* b1; float* w2; float* b2;
  float* loss;
  int R, N0, N1, N2;
  float alpha;
};
// Whether the shape fits the one-workgroup step (activations in 64 KB of LDS).
bool mlp2_step_ok(int64_t R, int64_t N0, int64_t N1, int64_t N2);
void mlp2_step(const Mlp2Step& a, hipStream_t s);
struct Lin1Fwd {
  const void* h; int64_t h_sm;
  const void* w; const void* b; const void* y;
  void* z; void* dz;
  int64_t R, N;
  float two_over_n;
};
void linear1_forward_mse(DType dt, const Lin1Fwd& a, hipStream_t s);
// The same with the layer's input h formed here from the previous GEMM's
// split-K partial sums: h = relu(sum of the splits in split order + hb),
// written to h_out (fp32, rows of N, N % 4 == 0, 16-byte aligned).
struct Lin1FwdParts {
  const float* part; int splits; int64_t plane;  // part[s * plane + r * N + k]
  const float* hb; float* h_out;
  const float* w; const float* b; const float* y;
  float* z; float* dz;
  int64_t R, N;
  float two_over_n;
};
void linear1_forward_mse_parts(const Lin1FwdParts& a, hipStream_t s);
// True when the plan for g computes a_rowsum_acc itself (the outer-product
// plan); otherwise the caller leaves it null and sums A on its own.
bool gemm_a_rowsum_fused(const Gemm& g);
// K splits of the launch's plan (1 when it has no split-K reduction).
int gemm_splits(const Gemm& g);
// Whether the skinny decode kernel takes this problem, and whether it can
// also normalise the A rows (layer norm over K, K <= 4096) while loading them.
bool gemm_is_skinny(const Gemm& g);
bool gemm_skinny_ln_ok(const Gemm& g);
// Packed decode weights: out[t][s][l][e] = W^T[16t + l%16][32s + 8(l/16) + e]
// for W^T [N][K] read through strides (s_n, s_k), zero-padded to whole
// 16-column tiles and 32-deep steps (packed_weight_elems elements).
int64_t packed_weight_elems(int64_t N, int64_t K);
void pack_weights(DType dt, const void* w, int64_t s_n, int64_t s_k, int64_t N, int64_t K, void* out,
                  hipStream_t s);
// Workspace bytes the launch needs (split-K partials); 0 when none.
size_t gemm_workspace_bytes(const Gemm& g);
void gemm(const Gemm& g, void* workspace, hipStream_t s);
// Two fp32 SGD weight updates (W += alpha A^T B with a bias row-sum
// accumulator each, same K) in one pack and one GEMM launch, when both take
// the outer-product plan; workspaces as gemm_workspace_bytes gives for each.
bool gemm_outer_pair_ok(const Gemm& g0, const Gemm& g1);
void gemm_outer_pair(const Gemm& g0, void* ws0, const Gemm& g1, void* ws1, hipStream_t s);

// How fp32 GEMMs compute: kF32Split3 splits each operand into bf16 hi + lo
// and accumulates hi*hi + hi*lo + lo*hi on bf16 MFMA in fp32 (default);
// kF32Native runs v_mfma_f32_32x32x2_f32.  `cfg` (-1 = heuristic) and
// `splits` (0 = heuristic) force a tile configuration for tuning sweeps.
enum F32Mode : int { kF32Split3 = 0, kF32Native = 1 };
constexpr int kMfConfigs = 11;  // tile configurations of the bf16-MFMA kernels
struct GemmTune {
  int f32_mode = kF32Split3;
  int cfg = -1;
  int splits = 0;
  bool no_skinny = false;  // route M <= 16 through gemm_mf too
  // split row panels finish their tiles in the kernel (no reduction launch);
  // APPLEGPU_SPLIT_INKERNEL=0 sends their sums to the reduction launch
  bool inkernel_splits = true;
};
GemmTune& gemm_tune();
// Name of the configuration the heuristic (or a forced tune) picks.
const char* gemm_plan_name(const Gemm& g);

// ── fused attention ───────────────────────────────────────────────────────
struct Attn {
  DType dt = DType::F32;
  int64_t B = 1, H = 1, Tq = 0, Tk = 0, D = 0;
  const void* q = nullptr; int64_t q_sb = 0, q_sh = 0, q_st = 0;  // unit d stride
  const void* k = nullptr; int64_t k_sb = 0, k_sh = 0, k_st = 0;
  const void* v = nullptr; int64_t v_sb = 0, v_sh = 0, v_st = 0;
  void* o = nullptr; int64_t o_sb = 0, o_sh = 0, o_st = 0;
  // fp32 MFMA kernel only: the output written instead as packed x3 rows of
  // the [B*Tq, H*D] matrix whose row is one query of one batch entry (heads
  // side by side), for a following packed-A GEMM (H*D % 16 == 0)
  void* o_pk = nullptr;
  bool causal = false;   // key j visible to query i iff j <= i (diagonal at (0,0))
  float scale = 1.f;
  // nsplit > 0 (2, 4 or 8; fp32): q, k, v point at split 0 of a split-K GEMM
  // workspace whose partial sums are `plane` elements apart; each value is
  // their sum (in split order) plus qb/kb/vb[h * b_sh + dim]
  int nsplit = 0;
  int64_t plane = 0, b_sh = 0;
  const void* qb = nullptr; const void* kb = nullptr; const void* vb = nullptr;
};
bool attention_supported(const Attn& a);
// Whether attention can read Q/K/V as projection partials (fp32 MFMA kernel:
// d = 64 or 128, 16-byte aligned rows).
bool attention_partials_ok(const Attn& a);
void attention(const Attn& a, hipStream_t s);

// ── KV-cache decode ───────────────────────────────────────────────────────
// Attention of Tq new query rows per (batch, head) over the first lens[b]
// rows of a [B, H, Tmax, D] cache whose last Tq valid rows are the queries'
// own keys: query row i sees keys j <= lens[b] - Tq + i.  lens is int32 [B]
// in device memory (clamped to [0, Tmax]).
struct DecodeAttn {
  DType dt = DType::F16;
  int64_t B = 1, H = 1, Tq = 1, Tmax = 0, D = 0;
  const void* q = nullptr; int64_t q_sb = 0, q_sh = 0, q_st = 0;  // unit d stride
  const void* k = nullptr; int64_t k_sb = 0, k_sh = 0, k_st = 0;
  const void* v = nullptr; int64_t v_sb = 0, v_sh = 0, v_st = 0;
  void* o = nullptr; int64_t o_sb = 0, o_sh = 0, o_st = 0;
  const int32_t* lens = nullptr;
  float scale = 1.f;
  // optional (Tq == 1): the step's new K and V rows [B, H, 1, D], stored as
  // cache row lens[b] - 1 by the same launch (and scored from registers)
  const void* kn = nullptr; int64_t kn_sb = 0, kn_sh = 0;
  const void* vn = nullptr; int64_t vn_sb = 0, vn_sh = 0;
};
bool decode_attention_supported(const DecodeAttn& a);
int decode_attention_splits(const DecodeAttn& a, int64_t* chunk);
size_t decode_attention_ws_bytes(const DecodeAttn& a);
void decode_attention(const DecodeAttn& a, void* ws, hipStream_t s);
// cache[b, h, pos[b] + t, :] = src[b, h, t, :] for t < T (rows that would
// land at or past Tmax are dropped); pos is int32 [B] in device memory.  A
// second (cache2, src2) pair of the same shape (the V cache beside the K
// cache) is written by the same launch.  Strides: (batch, head, token), unit
// stride along D.
struct KvWrite {
  DType dt = DType::F16;
  int64_t B = 1, H = 1, T = 0, D = 0, Tmax = 0;
  void* cache = nullptr; int64_t cs[3] = {0, 0, 0};
  const void* src = nullptr; int64_t xs[3] = {0, 0, 0};
  void* cache2 = nullptr; int64_t c2s[3] = {0, 0, 0};
  const void* src2 = nullptr; int64_t x2s[3] = {0, 0, 0};
  const int32_t* pos = nullptr;
};
void kv_write(const KvWrite& a, hipStream_t s);
// o = x elementwise with dtype conversion, o written through the strides of
// `so` (shape and destination strides) and x read through `sx`.
void copy_strided(DType in, DType out, const void* x, const ND& sx, void* o, const ND& so, hipStream_t s);

}  // namespace k
}  // namespace agpu
