/*
 * applegpu_ffi.h — C ABI of the MI355X (gfx950) backend for applegpu-runtime.
 *
 * Part 1 declares, with identical C signatures, every symbol of the
 * reference header backend_cpp/applegpu_ffi.h:11-92 (graph path
 * applegpu_ffi_*, eager path applegpu_eager_*), plus the exported-but-
 * undeclared applegpu_eager_execute_graph (crates/core/src/eager_ffi.rs:661-708).
 * Conventions are the reference's (crates/core/src/eager_ffi.rs:38-46,
 * backend_ffi.rs:26-34):
 *   - pointer-returning ops return the output's data pointer (base + byte
 *     offset) or NULL on failure; u64 id returns use 0 for failure; i32
 *     returns use 0 for success and -1 for failure; dtype returns -1 for an
 *     unknown id;
 *   - on failure a thread-local C string is set (applegpu_eager_last_error /
 *     applegpu_ffi_last_error), valid until the next error on that thread;
 *   - *out_id is written only on success;
 *   - dtype wire codes: 0 f32, 1 f16, 2 f64, 3 i8, 4 i16, 5 i32, 6 i64, 7 u8,
 *     8 u32, 9 bool, 10 bf16 (crates/core/src/tensor.rs:59-90);
 *   - shapes have at most 8 dims; one global lock serialises all calls.
 *
 * Memory: returned data pointers are HBM device pointers on MI355X (the
 * reference's were host-coherent Metal shared buffers).  Host reads and writes
 * go through the copy entry points in Part 2; setting APPLEGPU_HOST_VISIBLE=1
 * before init makes every allocation pinned host memory that both sides can
 * dereference (slow; compatibility only).
 *
 * Part 2 declares the additions this backend needs for the hot path; each
 * names the reference interface it replaces.
 */
#ifndef APPLEGPU_FFI_H
#define APPLEGPU_FFI_H

#include <stdint.h>
#include <stdbool.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ════════════════════ Part 1: reference surface ════════════════════════ */

/* Lifecycle */
bool applegpu_ffi_init(void);
const char* applegpu_ffi_last_error(void);

/* Allocation */
uint8_t* applegpu_ffi_alloc(uint64_t size_bytes, int8_t dtype_i8, uint64_t* out_tensor_id);
void applegpu_ffi_free(uint64_t tensor_id);

/* Tensor metadata */
int32_t applegpu_ffi_register_tensor(uint64_t tensor_id, const uint64_t* dims, uint32_t ndim, int8_t dtype_i8);
int32_t applegpu_ffi_shape(uint64_t tensor_id, uint64_t* out_dims, uint32_t* out_ndim);
int8_t applegpu_ffi_dtype(uint64_t tensor_id);

/* Ops (return output tensor_id, 0 on failure) */
uint64_t applegpu_ffi_add(uint64_t a_id, uint64_t b_id);
uint64_t applegpu_ffi_matmul(uint64_t a_id, uint64_t b_id);
uint64_t applegpu_ffi_relu(uint64_t input_id);
uint64_t applegpu_ffi_mul(uint64_t a_id, uint64_t b_id);
uint64_t applegpu_ffi_sub(uint64_t a_id, uint64_t b_id);
uint64_t applegpu_ffi_neg(uint64_t input_id);
int32_t applegpu_ffi_copy(uint64_t src_id, uint64_t dst_id);

/* Ops with output allocation (return data_ptr, write tensor_id to *out_id) */
uint8_t* applegpu_ffi_add_out(uint64_t a_id, uint64_t b_id, uint64_t* out_id);
uint8_t* applegpu_ffi_mul_out(uint64_t a_id, uint64_t b_id, uint64_t* out_id);
uint8_t* applegpu_ffi_sub_out(uint64_t a_id, uint64_t b_id, uint64_t* out_id);
uint8_t* applegpu_ffi_matmul_out(uint64_t a_id, uint64_t b_id, uint64_t* out_id);
uint8_t* applegpu_ffi_relu_out(uint64_t input_id, uint64_t* out_id);
uint8_t* applegpu_ffi_neg_out(uint64_t input_id, uint64_t* out_id);
uint8_t* applegpu_ffi_div_out(uint64_t a_id, uint64_t b_id, uint64_t* out_id);
uint8_t* applegpu_ffi_threshold_backward_out(uint64_t grad_id, uint64_t input_id, float threshold, uint64_t* out_id);
uint8_t* applegpu_ffi_scalar_mul_out(uint64_t input_id, float scale, uint64_t* out_id);
uint8_t* applegpu_ffi_mean_all_out(uint64_t input_id, uint64_t* out_id);

/* Eval / sync */
int32_t applegpu_ffi_eval(uint64_t tensor_id);
void applegpu_ffi_synchronize(void);

/* Readback */
int32_t applegpu_ffi_read_f32(uint64_t tensor_id, float* out_ptr, uint64_t max_elements);

/* ── Eager dispatch (bypasses graph engine) ── */
bool applegpu_eager_init(void);
const char* applegpu_eager_last_error(void);

uint8_t* applegpu_eager_alloc(const uint64_t* dims, uint32_t ndim, int8_t dtype, uint64_t* out_id);
void applegpu_eager_free(uint64_t id);
int32_t applegpu_eager_register_shape(uint64_t id, const uint64_t* dims, uint32_t ndim);
int32_t applegpu_eager_shape(uint64_t id, uint64_t* out_dims, uint32_t* out_ndim);
int8_t applegpu_eager_dtype(uint64_t id);

uint8_t* applegpu_eager_add(uint64_t a_id, uint64_t b_id, uint64_t* out_id);
uint8_t* applegpu_eager_sub(uint64_t a_id, uint64_t b_id, uint64_t* out_id);
uint8_t* applegpu_eager_mul(uint64_t a_id, uint64_t b_id, uint64_t* out_id);
uint8_t* applegpu_eager_div(uint64_t a_id, uint64_t b_id, uint64_t* out_id);
uint8_t* applegpu_eager_relu(uint64_t input_id, uint64_t* out_id);
uint8_t* applegpu_eager_neg(uint64_t input_id, uint64_t* out_id);
uint8_t* applegpu_eager_matmul(uint64_t a_id, uint64_t b_id, uint64_t* out_id);
uint8_t* applegpu_eager_matmul_ex(uint64_t a_id, uint64_t b_id, bool transpose_a, bool transpose_b, uint64_t* out_id);

uint8_t* applegpu_eager_threshold_backward(uint64_t grad_id, uint64_t input_id, float threshold, uint64_t* out_id);
uint8_t* applegpu_eager_scalar_mul(uint64_t input_id, float scale, uint64_t* out_id);
uint8_t* applegpu_eager_mean_all(uint64_t input_id, uint64_t* out_id);

uint8_t* applegpu_eager_sum_dim(uint64_t input_id, int64_t dim, bool keepdim, uint64_t* out_id);

uint8_t* applegpu_eager_create_view(uint64_t base_id, const uint64_t* shape, const uint64_t* strides, uint32_t ndim, uint64_t offset, uint64_t* out_id);

int32_t applegpu_eager_add_inplace(uint64_t self_id, uint64_t other_id);
int32_t applegpu_eager_add_scaled_inplace(uint64_t self_id, uint64_t other_id, float alpha);

void applegpu_eager_flush_and_wait(void);
void applegpu_eager_synchronize(void);

/* GPT-2 ops */
uint8_t* applegpu_eager_embedding(uint64_t weight_id, uint64_t indices_id, uint64_t* out_id);
uint8_t* applegpu_eager_layer_norm(uint64_t input_id, uint64_t gamma_id, uint64_t beta_id, float eps, uint64_t* out_id);
uint8_t* applegpu_eager_gelu(uint64_t input_id, uint64_t* out_id);
uint8_t* applegpu_eager_softmax(uint64_t input_id, uint64_t* out_id);

/* Reverse lookup: find tensor_id by buffer data pointer. Returns 0 if not found. */
uint64_t applegpu_eager_find_by_data_ptr(const uint8_t* ptr);

/* Exported but undeclared in the reference (eager_ffi.rs:661-708; bound via
 * ctypes in python/applegpu_runtime/compile_backend.py:961-1030): runs a
 * serialized torch.compile FX graph.  ops_data is the op list of
 * crates/core/src/compiled_graph.rs:7-9 (per op: code u8, n_inputs u8,
 * inputs u16[n], out_ndim u8, out_dims u64[ndim], out_dtype u8,
 * params_len u8, params f32[plen]; codes 0-13 and 255 of
 * compiled_graph.rs:43-57); node i < n_inputs is input_tids[i], each op
 * appends one node.  Writes the id and data pointer of node
 * output_indices[i] to out_tids[i] / out_ptrs[i]: an input (or its
 * identity) comes back as its own id, every other returned node as a new id
 * the caller frees, one id per node.  The ops are queued on the library
 * stream (addmm + relu and other GEMM epilogues fuse); contents are valid
 * after flush_and_wait or to any later op.  Returns n_outputs, or -1 with
 * "compiled graph failed: ..." set (a malformed op list is rejected before
 * anything runs). */
int32_t applegpu_eager_execute_graph(const uint8_t* ops_data, uint32_t ops_len,
                                     const uint64_t* input_tids, uint32_t n_inputs,
                                     const uint16_t* output_indices, uint32_t n_outputs,
                                     uint64_t* out_tids, uint8_t** out_ptrs);

/* ════════════════════ Part 2: MI355X additions ═════════════════════════ */

/* Generic lazy op: records op `op` (a name of the Python surface: "softmax",
 * "layer_norm", "attention_causal", "quantize_per_row", ...) on the given
 * input ids with float/int parameters; writes up to max_out new ids and
 * returns their number, or -1 (error in applegpu_ffi_last_error).
 * Replaces the PyO3 module's BACKEND.<op> calls (crates/python/src/lib.rs:830-1258,
 * Backend trait crates/python/src/backend.rs:17-204) into LazyRuntime ops
 * (crates/core/src/ops.rs). */
int32_t applegpu_graph_op(const char* op, const uint64_t* inputs, uint32_t n_inputs,
                          const double* fparams, uint32_t n_f, const int64_t* iparams, uint32_t n_i,
                          uint64_t* out_ids, uint32_t max_out);

/* Host <-> device copies for the graph path: write_bytes replaces the host
 * memcpy into a shared buffer behind from_numpy/from_bytes
 * (crates/python/src/lib.rs:419-512); read_bytes evaluates a pending tensor
 * and copies its logical (row-major) bytes out, replacing
 * LazyRuntime::read_bytes behind to_numpy (crates/python/src/lib.rs:140-160).
 * nbytes must equal numel * element size. */
int32_t applegpu_ffi_write_bytes(uint64_t tensor_id, const void* src, uint64_t nbytes);
int32_t applegpu_ffi_read_bytes(uint64_t tensor_id, void* dst, uint64_t nbytes);
/* 1 when the tensor still has unevaluated ops, 0 when materialised, -1 unknown. */
int32_t applegpu_ffi_is_pending(uint64_t tensor_id);
/* Element strides of a tensor (views are strided). */
int32_t applegpu_ffi_strides(uint64_t tensor_id, int64_t* out_strides, uint32_t* out_ndim);

/* Runtime introspection and setters of the Python surface: pool_stats,
 * pool_drain, set_pool_watermark, memory_usage, tensor_count, set_limits,
 * device_name (crates/python/src/lib.rs:386-395, 788-806, 1136-1151;
 * crates/core/src/pool.rs:7-12, limits.rs:39-77).
 * out[0..5] = hits, misses, pooled_bytes, bucket_count, live_bytes. */
int32_t applegpu_ffi_pool_stats(uint64_t* out5);
void applegpu_ffi_pool_drain(void);
void applegpu_ffi_set_pool_watermark(uint64_t bytes);
uint64_t applegpu_ffi_memory_usage(void);
uint64_t applegpu_ffi_tensor_count(void);
void applegpu_ffi_set_limits(uint64_t max_tensor_bytes, uint64_t max_memory_bytes, uint64_t max_tensors);
int32_t applegpu_ffi_device_name(char* out, uint32_t cap);
/* out[0..4] = evals, nodes, fused GEMM epilogues, launches saved by fusion */
int32_t applegpu_ffi_graph_stats(uint64_t* out4);
/* The same counters and more, for the lazy executor's fusion pass
 * (crates/core/src/fusion.rs:243-282 replaces chains of elementwise nodes
 * by one fused node; the reference exposes no counters for it): writes up
 * to `cap` of evals, nodes, fused GEMM epilogues, launches saved, fused
 * elementwise chains, nodes inside those chains, kernel launcher calls;
 * returns the number of counters available (7). */
uint32_t applegpu_ffi_graph_stats_ex(uint64_t* out, uint32_t cap);
/* Test hook (no reference counterpart): the next n device allocations fail,
 * so the out-of-memory path can be exercised from the host. */
void applegpu_ffi_inject_alloc_failures(int32_t n);
/* Measurement (no reference counterpart; the reference times with
 * time.perf_counter around a flush, benchmarks/bench_mlp_cpp.py:39-45):
 * record a HIP event in slot 0..15 on the library's stream, and the elapsed
 * milliseconds between two recorded slots (waits for the later one). */
int32_t applegpu_ffi_event_record(uint32_t slot);
float applegpu_ffi_event_elapsed_ms(uint32_t start_slot, uint32_t end_slot);

/* Graph capture (no reference counterpart; the reference re-encodes every op
 * of every eval into a Metal command buffer, crates/core/src/lazy.rs:369-474,
 * crates/core/src/compute.rs:2598-2698).  capture_begin starts recording the
 * library's stream: ops issued until capture_end (eager ops, and the kernels
 * of lazy evals run in between) are recorded instead of executed, into a
 * HIP graph whose handle (> 0) capture_end returns (-1 on failure).  Every
 * buffer allocated during the capture belongs to the graph until
 * graph_destroy: graph_replay (asynchronous, on the library stream)
 * recomputes the same ops from the current contents of their inputs into
 * the same output buffers.  While capturing, host reads/writes of tensors,
 * read_f32 and event_elapsed_ms fail and synchronize returns at once;
 * capture_abort ends a capture and drops what it recorded.  Calls that
 * overlap on one stream race like any other work on it. */
/* KV-cache append for decode (replaces the reference's per-step concat of
 * the whole cache, python/applegpu_runtime/models/gpt2.py:122-126, which
 * copies every earlier K/V row again at each step): cache is a [B, H, Tmax, D]
 * tensor (or view) with unit stride along D, rows is [B, H, T, D] of the same
 * dtype, pos is int32 [B] in device memory.  Writes
 * cache[b, h, pos[b] + t, :] = rows[b, h, t, :] in place, on the library
 * stream; rows whose position falls outside [0, Tmax) are not written.  The
 * positions are read by the kernel, not the host, so the call can sit inside
 * a captured graph that is replayed with advancing positions.  The matching
 * reader is the lazy op "decode_attention" (applegpu_graph_op): inputs q
 * [B, H, Tq, D], k_cache, v_cache [B, H, Tmax, D] and lens int32 [B]; query
 * row i of sequence b attends to cache rows j <= lens[b] - Tq + i.  With
 * Tq == 1 it takes two more inputs, k_new and v_new [B, H, 1, D]: the step's
 * own rows, which the same launch stores as cache row lens[b] - 1 (when
 * 1 <= lens[b] <= Tmax) and attends to, in place of this call.
 * Returns 0, or -1 with the error set. */
int32_t applegpu_kv_write(uint64_t cache_id, uint64_t rows_id, uint64_t pos_id);
/* The K and V appends of one layer in one launch: same contract as
 * applegpu_kv_write for (k_cache, k_rows) and (v_cache, v_rows), which must
 * have the same shapes and dtype. */
int32_t applegpu_kv_write_pair(uint64_t k_cache_id, uint64_t v_cache_id, uint64_t k_rows_id, uint64_t v_rows_id,
                               uint64_t pos_id);

int32_t applegpu_capture_begin(void);
int64_t applegpu_capture_end(void);
int32_t applegpu_capture_abort(void);
int32_t applegpu_graph_replay(int64_t handle);
int32_t applegpu_graph_destroy(int64_t handle);
/* Device bytes the graph's buffers occupy (0 for an unknown handle). */
uint64_t applegpu_graph_bytes(int64_t handle);

/* GEMM tuning (no reference counterpart; the reference chooses between
 * MPSMatrixMultiplication and its tiled kernel inside
 * swift/Sources/AppleGPUBridge/compute.swift:1544-1630).  f32_mode: 0 = fp32
 * operands split into bf16 hi/lo with three bf16 MFMAs per product (default),
 * 1 = native fp32 MFMA (v_mfma_f32_32x32x2_f32; also APPLEGPU_GEMM_F32=native).
 * cfg: -1 = heuristic, 0..10 = tile configuration (BM x BN x BK: 128x128x32,
 * 64x128x32, 64x64x64, 32x64x64, 32x32x64, 128x128x64, 64x64x64, 64x128x64,
 * 32x32x256, 32x64x256, 64x64x128); for fp32 weights packed by pack_weight_x3:
 * 0 = 128x64 split tiles, 1 = 128x32 split tiles, 2 = 32x32 row panels,
 * 3 = 128x128 weight-streaming panels (packed activation rows).
 * splits: 0 = heuristic, n = split K across n blocks.
 * Returns 0, or -1 for an out-of-range value. */
int32_t applegpu_ffi_gemm_tune(int32_t f32_mode, int32_t cfg, int32_t splits);
/* GEMMs with at most 16 rows of A (decode steps) run a weight-streaming
 * kernel instead of the MFMA tiles unless this is switched off (enable = 0;
 * also APPLEGPU_GEMM_SKINNY=0) or a cfg/splits tune is forced.  Returns the
 * previous setting (1 = on).  No reference counterpart (tuning). */
int32_t applegpu_ffi_gemm_skinny(int32_t enable);
/* Split-K packed-A row panels (fp32 GPT-2 projections) finish each output
 * tile in the GEMM launch itself, by whichever split of the tile arrives
 * last, instead of in a separate reduction launch, unless this is switched
 * off (enable = 0; also APPLEGPU_SPLIT_INKERNEL=0).  Both give the same bits.
 * Returns the previous setting (1 = on).  No reference counterpart (tuning;
 * it replaces nothing the reference has). */
int32_t applegpu_ffi_split_inkernel(int32_t enable);
/* 1 when an M x K (packed rows) by K x N (packed fp32 weights) product runs
 * a row-panel plan that writes its output, packed rows and row statistics
 * in one launch (so a layer_norm of its output can fold into the next
 * projection), 0 when not, -1 on bad extents.  No reference counterpart
 * (plan introspection). */
int32_t applegpu_ffi_x3_rows_out(int64_t M, int64_t N, int64_t K);
/* Evaluates several lazy tensors in one fusion-planned walk (a producer
 * whose outputs are read by more than one of them, such as a GEMM writing
 * its output, its packed rows and its row statistics, then runs once).  No
 * reference counterpart: the reference's lazy eval takes one root
 * (crates/core/src/lazy.rs:208-474); this is the multi-root walk that
 * applegpu_eager_execute_graph runs for a graph's outputs.  Returns 0, or -1
 * with the error set. */
int32_t applegpu_ffi_eval_many(const uint64_t* tensor_ids, uint32_t n);
/* The plan the GEMM heuristic picks for an M x N x K (batch) problem of the
 * given dtype and operand layouts (a_kcontig: A(m,k) has unit k stride;
 * b_kcontig: B(k,n) has unit k stride), written as text into out. */
int32_t applegpu_ffi_gemm_plan(int64_t M, int64_t N, int64_t K, int64_t batch, int8_t dtype_i8,
                               bool a_kcontig, bool b_kcontig, char* out, uint32_t cap);

/* Generic eager op: runs `op` at once (same names and parameters as
 * applegpu_graph_op), registers the outputs, writes their ids to out_ids and
 * returns their number (or -1).  Replaces the aten kernels of the
 * PrivateUse1 shim that the reference runs through CPU fallback or several
 * eager calls (backend_cpp/applegpu_backend.cpp:753-764 masked ops,
 * :801-867 mse_loss, :943-951 softmax, :1055-1096 registrations).  The
 * training-step ops sgd_matmul_ (w, a, b[, bias]), sgd_sum_rows_ (bias, g),
 * linear_backward_sgd_ (w, b, g, a[, mask]) and linear_mse_backward_sgd_
 * (h, w, b, y; iparams[0]: return the input gradient) update their
 * parameters in place; fparams[0] is the step's alpha (-lr).  They run
 * eagerly only (applegpu_graph_op refuses them). */
int32_t applegpu_eager_op(const char* op, const uint64_t* inputs, uint32_t n_inputs,
                          const double* fparams, uint32_t n_f, const int64_t* iparams, uint32_t n_i,
                          uint64_t* out_ids, uint32_t max_out);

/* Host <-> device copies for eager tensors (any strides on the device side):
 * replace the shim's host memcpy on shared buffers in copy_/_copy_from
 * (backend_cpp/applegpu_backend.cpp:267-341). nbytes = numel * element size. */
int32_t applegpu_eager_copy_from_host(uint64_t id, const void* src, uint64_t nbytes);
int32_t applegpu_eager_copy_to_host(uint64_t id, void* dst, uint64_t nbytes);
/* dst = src on the device (dtype cast allowed, dst of any strides): replaces
 * the scalar_mul(view, 1.0) + storage swap copy idiom
 * (backend_cpp/applegpu_backend.cpp:274-299). */
int32_t applegpu_eager_copy_(uint64_t dst_id, uint64_t src_id);
/* Fill with a value on the device (any strides): replaces the CPU memset of
 * fill_/zero_ (backend_cpp/applegpu_backend.cpp:729-751). */
int32_t applegpu_eager_fill(uint64_t id, double value);
/* Data pointer (buffer base + byte offset) of an eager tensor, evaluating it
 * first if it is pending; NULL for an unknown id.  The pointer-returning
 * eager calls give it directly; this serves ids returned by applegpu_eager_op
 * (the reference's eager ops return it with the id, eager_ffi.rs:234-262). */
uint8_t* applegpu_eager_data_ptr(uint64_t id);
/* A view of base's storage read as dtype `dtype_i8`, with element strides and
 * a byte offset from base's data (bounds-checked against the allocation):
 * maps a torch tensor (storage, dtype, storage offset, strides) exactly.
 * Replaces resolve_tensor_id's create_view (backend_cpp/applegpu_backend.cpp:
 * 37-93), whose views keep the storage's registration dtype. */
uint8_t* applegpu_eager_view_typed(uint64_t base_id, const uint64_t* shape, const uint64_t* strides, uint32_t ndim,
                                   uint64_t offset_bytes, int8_t dtype_i8, uint64_t* out_id);
/* y = act(x W^T + b) in one GEMM with a fused epilogue (act: 0 none, 1 relu,
 * 2 gelu-tanh, 3 gelu-erf; bias_id 0 = none): replaces addmm's W^T copy +
 * matmul + bias add (backend_cpp/applegpu_backend.cpp:584-620). */
uint8_t* applegpu_eager_linear(uint64_t x_id, uint64_t w_id, uint64_t bias_id, int32_t act, uint64_t* out_id);
/* Allocation-free linear: no counterpart in the reference.  For callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc): out = act(x W^T + b) as
 * applegpu_eager_linear computes it (the same kernels and results wherever
 * the same plan fits, see below), written
 * into the caller's contiguous [M, N] tensor `out_id` of x's dtype.  x [M, K],
 * weight [N, K] and the optional contiguous bias [N] (bias_id 0 = none) must
 * already hold values, and out may not share storage with them.  The GEMM's
 * split-K partial sums go to a static 64 MiB device array that each GPU the
 * library runs on holds until the process ends.  A product whose default
 * plan packs its operands into more workspace than that (the fp32
 * outer-product plan, (M + N) K 4 bytes) takes a plan that fits instead
 * (results then agree with applegpu_eager_linear to the fp32 GEMM bar, not
 * bit for bit); one whose split-K partials would exceed it (only reachable
 * through a forced applegpu_ffi_gemm_tune split count: the planner's own
 * split choices stay below it) is rejected with an error.  Every call on one
 * GPU shares
 * that array and it keeps the last call's partials; calls are ordered on
 * the library's one stream, but work that overlaps them on one GPU from
 * another stream would race on it.  Nothing in it needs to start at zero:
 * each split writes its whole partial tile before the reduction reads it.
 * Returns 0, or -1 with the error set. */
int32_t applegpu_eager_linear_noalloc(uint64_t x_id, uint64_t w_id, uint64_t bias_id, int32_t act,
                                      uint64_t out_id);
/* C = op(A) op(B) with a fused "mask" epilogue: out = (mask > 0) ? A@B : 0,
 * i.e. matmul followed by threshold_backward(., mask, 0) in one kernel
 * (eager.rs:485-560 + eager.rs:775-818). */
uint8_t* applegpu_eager_matmul_masked(uint64_t a_id, uint64_t b_id, bool transpose_a, bool transpose_b,
                                      uint64_t mask_id, uint64_t* out_id);
/* loss = mean((a-b)^2) as one fused reduction, and its gradient
 * (a-b) * 2/n * g: replace the shim's sub/mul/mean_all decomposition
 * (backend_cpp/applegpu_backend.cpp:801-867). */
uint8_t* applegpu_eager_mse_loss(uint64_t a_id, uint64_t b_id, uint64_t* out_id);
uint8_t* applegpu_eager_mse_loss_backward(uint64_t grad_id, uint64_t a_id, uint64_t b_id, uint64_t* out_id);
/* Element strides of an eager tensor. */
int32_t applegpu_eager_strides(uint64_t id, int64_t* out_strides, uint32_t* out_ndim);

#ifdef __cplusplus
}
#endif

#endif /* APPLEGPU_FFI_H */
