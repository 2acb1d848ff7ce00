// Op table and the lazy graph executor.
//
// Every op of the Python surface has a name in one table; `run_op` executes
// it at once (eager path) or, in meta mode, only validates it and returns an
// output description (lazy recording).  `eval` materialises a pending tensor:
// post-order walk of its pending ancestors, fusion planning, then one launch
// sequence on the runtime stream.
//
// Reference: LazyRuntime::record_op / eval / eval_single_cb
// (crates/core/src/lazy.rs:148, 208-474), Graph::topo_sort
// (crates/core/src/graph.rs:541), fusion::optimize (crates/core/src/fusion.rs:243-282).
#pragma once

#include <string>
#include <vector>

#include "core.hpp"

namespace agpu {

struct Node {
  int code = 0;
  std::vector<TensorP> in;
  std::vector<double> f;
  std::vector<int64_t> iv;
  // Multi-output producers: the pending outputs to fill when it runs.
  std::vector<std::weak_ptr<Tensor>> selectors;
};

// Meta mode: ops validate and describe their outputs without touching the GPU.
bool meta_mode();
struct MetaScope {
  MetaScope();
  ~MetaScope();
  bool prev;
};

int op_code(const char* name);  // -1 when unknown
const char* op_name(int code);
int op_outputs(int code);       // number of outputs (1 or 2)

// Execute (or, in meta mode, describe) an op.
std::vector<TensorP> run_op(int code, const std::vector<TensorP>& in, const std::vector<double>& f,
                            const std::vector<int64_t>& iv);

// Lazy recording: validates, returns pending output tensors.
std::vector<TensorP> record_op(int code, const std::vector<TensorP>& in, const std::vector<double>& f,
                               const std::vector<int64_t>& iv);

// Materialise a pending tensor (no-op when it already has storage).
void eval(const TensorP& t);
// Materialise several pending tensors with one fusion plan over all their
// pending ancestors (a node shared by two roots runs once).
void eval_all(const std::vector<TensorP>& roots);

// torch.compile bytecode executor (crates/core/src/compiled_graph.rs:61-193):
// runs a serialized FX graph over the eager tensors `inputs` and returns
// the ids and data pointers of the nodes `out_idx` names.  Throws on a
// malformed graph or a failing op; nothing is written to the outputs then.
void execute_compiled(const uint8_t* ops, size_t len, const uint64_t* inputs, uint32_t n_in, const uint16_t* out_idx,
                      uint32_t n_out, uint64_t* out_ids, uint8_t** out_ptrs);

struct GraphStats {
  uint64_t evals = 0, nodes = 0, fused_gemm_epilogues = 0, launches_saved = 0;
  uint64_t fused_chains = 0, chain_nodes = 0;  // elementwise chains run as one launch, and their nodes
  uint64_t launcher_calls = 0;                  // kernel launcher calls (one per launched kernel family)
};
GraphStats graph_stats();

}  // namespace agpu
