// Internal declarations of the MI355X plugin execution provider.
//
// Layering (reference counterparts in parentheses):
//   ep.cpp     C-ABI entry points, factory / EP / node-compute-info vtables,
//              hipMalloc allocator and data transfer (rust/src/lib.rs,
//              rust/src/factory.rs, rust/src/ep.rs:48-113, 1878-2171)
//   graph.cpp  reading an OrtGraph into an owned IR, claim predicates and
//              convex clustering (rust/src/registry.rs, rust/src/ep.rs:119-895)
//   plan.cpp   per-fused-node plan: initializers copied to HBM once, topological
//              op list, shape inference and kernel launches at Compute
//              (rust/src/ep.rs:928-1298, rust/src/engine.rs)
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../../include/ort_plugin_ep_abi.h"

namespace ortmi_ep {

// ------------------------------------------------------------------ errors --
struct EpError : std::runtime_error {
    OrtErrorCode code;
    EpError(OrtErrorCode c, const std::string& m) : std::runtime_error(m), code(c) {}
};
[[noreturn]] inline void fail(const std::string& msg, OrtErrorCode c = ORT_EP_FAIL) {
    throw EpError(c, msg);
}
// Throw on a non-null OrtStatus returned by the host, releasing it first.
void check_ort(const OrtApi* api, OrtStatus* st, const char* what);
void check_hip(hipError_t e, const char* what);
void check_kernel(int rc, const char* what);

// ---------------------------------------------------------------------- IR --
struct Attr {
    OrtOpAttrType type = ORT_OP_ATTR_UNDEFINED;
    int64_t i = 0;
    float f = 0.f;
    std::string s;
    std::vector<int64_t> ints;
    std::vector<float> floats;
};

struct ValueDesc {
    std::string name;
    int dtype = 0;                 // ONNXTensorElementDataType
    std::vector<int64_t> dims;     // -1 for symbolic
    bool has_shape = false;
    bool is_initializer = false;
    std::vector<uint8_t> data;     // initializer bytes (copied at read time)
};

struct NodeDesc {
    size_t id = 0;
    std::string name, op, domain;
    int since_version = 0;
    std::vector<std::string> inputs;   // "" = absent optional input
    std::vector<std::string> outputs;  // "" = absent optional output
    std::map<std::string, Attr> attrs;
    const OrtNode* handle = nullptr;   // valid during GetCapability / Compile only

    int64_t attr_int(const char* k, int64_t dflt) const {
        auto it = attrs.find(k);
        return it == attrs.end() ? dflt : it->second.i;
    }
    float attr_float(const char* k, float dflt) const {
        auto it = attrs.find(k);
        return it == attrs.end() ? dflt : it->second.f;
    }
    std::string attr_str(const char* k, const std::string& dflt) const {
        auto it = attrs.find(k);
        return it == attrs.end() ? dflt : it->second.s;
    }
    bool has_input(size_t i) const { return i < inputs.size() && !inputs[i].empty(); }
};

struct GraphIR {
    std::vector<NodeDesc> nodes;                 // graph order
    std::map<std::string, ValueDesc> values;     // every named value seen
    std::vector<std::string> inputs, outputs;    // graph inputs / outputs
};

// Read a whole OrtGraph (nodes, value infos, initializer bytes, attributes).
GraphIR read_graph(const OrtApi* api, const OrtGraph* graph);

// ------------------------------------------------------------- op registry --
// Claim predicate: returns "" when the node is supported, else the reason.
using ClaimFn = std::string (*)(const NodeDesc&, const GraphIR&);
ClaimFn find_claim(const std::string& domain, const std::string& op);
std::string claim_reason(const NodeDesc& n, const GraphIR& g);  // "" = claimed

// Partition the claimed nodes into convex, acyclic clusters (each becomes one
// fused node). Returns node indices (into g.nodes) per cluster, topologically
// ordered inside each cluster.
std::vector<std::vector<size_t>> build_clusters(const GraphIR& g, const std::vector<bool>& claimed);

// ------------------------------------------- layer groups of large decoders --
// (rust/src/ep.rs:296-516, README.md "Large-decoder partition metadata")
// Model metadata key whose value is a JSON array of residual output names, one
// per transformer layer; it takes precedence over inference.
constexpr const char* kLayerBoundaryKey = "onnxruntime_ep_mlx.layer_boundary_outputs";
// Parse a JSON array of strings (the metadata value); false if it is anything else.
bool parse_json_string_array(const std::string& text, std::vector<std::string>* out);
// Residual outputs that end each layer, inferred from data flow: between two
// consecutive decoder-attention nodes (PagedAttention, or GroupQueryAttention /
// MultiHeadAttention / Attention with present key and value outputs) the last
// Add that the first reaches and that reaches the second. Empty when any pair
// has no such Add or there are fewer than two attention nodes.
std::set<std::string> infer_layer_boundaries(const GraphIR& g);
// Layers per partition from the ONNXRUNTIME_EP_MLX_LAYER_PARTITIONS value; 0 keeps
// every cluster whole. Unset, empty or "auto" keeps decoders whole on MI355X (the
// one-launch decode step needs the whole decoder in one fused node); "0", "off",
// "false" disable; a positive integer is the span; anything else disables.
size_t select_layer_span(const char* value);
// Cut each cluster (in its topological order) after every `span`-th node that
// produces a boundary output.
std::vector<std::vector<size_t>> split_layer_clusters(const GraphIR& g,
                                                      std::vector<std::vector<size_t>> clusters,
                                                      const std::set<std::string>& boundaries,
                                                      size_t span);

// Compile-time rewrites of a fused node's subgraph (SwiGLU, and with
// decode_fusions the QKV / gate-up merges and norm prologues).
void fuse_subgraph(GraphIR& g, const std::vector<std::string>& outputs, bool decode_fusions);

// ------------------------------------------------------------------- plan --
struct DeviceBuffer {
    void* ptr = nullptr;
    size_t bytes = 0;
    ~DeviceBuffer();
};

// Compiled form of one fused node.
class Plan {
   public:
    Plan(GraphIR sub, std::vector<std::string> inputs, std::vector<std::string> outputs,
         int device);
    ~Plan();
    // Run with the fused node's kernel context.
    void compute(const OrtApi* api, OrtKernelContext* ctx);
    const std::vector<std::string>& input_names() const { return inputs_; }
    const std::vector<std::string>& output_names() const { return outputs_; }

   private:
    struct Tensor {
        void* ptr = nullptr;
        int dtype = 0;
        std::vector<int64_t> dims;
        // splits > 0: the value is a one-token attention output still held as fp32
        // split partials [heads][splits][head + 2] (see the attention-merge rewrite).
        int64_t splits = 0;
        int64_t head = 0;
        // Host-memory input: `ptr` is its device staging buffer and `host` the
        // caller's buffer. lazy: the staging copy is left to the consumer (GQA
        // past KV uploads only its valid rows).
        const void* host = nullptr;
        bool lazy = false;
        int64_t numel() const {
            int64_t n = 1;
            for (auto d : dims) n *= d;
            return n;
        }
    };
    // Launch signature of one input: its device address (null for host inputs,
    // which are staged into a fixed buffer), element type and shape.
    struct InputSig {
        const void* ptr = nullptr;
        int dtype = 0;
        std::vector<int64_t> dims;
        bool operator==(const InputSig& o) const {
            return ptr == o.ptr && dtype == o.dtype && dims == o.dims;
        }
    };
    // A host scalar a captured graph depends on: 1 <= value <= hi.
    struct Guard {
        std::string name;
        int64_t hi = 0;
    };
    struct OutputRec {
        size_t index = 0;
        std::vector<int64_t> dims;
        void* ptr = nullptr;
    };

    void* arena_alloc(size_t bytes);
    void* workspace(size_t bytes);
    Tensor& out_tensor(const std::string& name, int dtype, const std::vector<int64_t>& dims,
                       const OrtApi* api, OrtKernelContext* ctx);
    // The caller's buffer of fused-node output `name` (host or device memory), or
    // null when `name` is not a fused-node output. `record` keeps the output for
    // the graph-replay bookkeeping (the decode program does not need it).
    void* output_buffer(const std::string& name, const std::vector<int64_t>& dims,
                        const OrtApi* api, OrtKernelContext* ctx, bool record = true);
    // Queue a device -> host copy of `rows` rows of `row_bytes` from each of
    // `slabs` slabs (pitch `pitch` bytes on both sides) after the run's kernels.
    void copy_out_rows(void* host, const void* dev, size_t pitch, size_t row_bytes, size_t rows,
                       size_t slabs);
    void run_node(const NodeDesc& n, const OrtApi* api, OrtKernelContext* ctx);
    int32_t host_i32(const std::string& name);
    void read_device_scalars();
    int32_t* scalar_host_ = nullptr;  // pinned landing slots of read_device_scalars
    size_t scalar_host_n_ = 0;
    bool guards_hold(const std::vector<Guard>& guards) const;
    bool replay(const OrtApi* api, OrtKernelContext* ctx);
    bool capture(const OrtApi* api, OrtKernelContext* ctx, const std::vector<InputSig>& sig);
    // One-launch decode step (ortmi_decoder_decode_step) for a fused node that is a
    // whole int4 decoder, at one-token steps on a device-resident shared KV cache.
    struct DecodeProgram;
    void match_decode_program();
    bool run_decode_program(const OrtApi* api, OrtKernelContext* ctx);
    std::unique_ptr<DecodeProgram> dprog_;
    bool dprog_required_ = false;  // ORTMI_EP_PROGRAM=require: fail when it does not apply
    int64_t dprog_fallbacks_ = 0;  // one-token steps the program did not complete (run op by op)
    std::string dprog_reject_ = "no decoder structure", dprog_ids_;  // why not; the ids input

    GraphIR sub_;
    std::vector<std::string> inputs_, outputs_;
    std::unordered_map<std::string, int> output_index_;
    std::map<std::string, std::unique_ptr<DeviceBuffer>> constants_;  // initializers in HBM
    std::unordered_map<std::string, Tensor> env_;                     // values of this run
    std::unordered_map<std::string, int32_t> host_scalars_;
    int device_ = 0;
    hipStream_t stream_ = nullptr;
    // Bump arena for intermediates, reset per Compute and grown on demand.
    std::vector<std::unique_ptr<DeviceBuffer>> arena_;
    size_t arena_off_ = 0;
    size_t arena_need_ = 0;
    std::unique_ptr<DeviceBuffer> workspace_;
    std::vector<std::unique_ptr<DeviceBuffer>> stage_;   // per input: host-input staging
    std::vector<std::pair<const void*, bool>> devptr_;   // per input: last pointer, is device
    std::vector<bool> lazy_input_;                      // per input: GQA past KV (staged lazily)
    std::mutex mu_;  // one Compute at a time per fused node (rust/src/ep.rs:1884-1889)

    // HIP-graph replay of a whole Compute. A run whose every launch is graph-safe
    // (no host round trip, no host-memory output, decode attention reading the
    // sequence length from device memory) marks its signature capturable; the
    // next run with the same signature is captured, later ones replay the graph.
    // Any device (re)allocation bumps mem_epoch_ and retires the graph.
    bool graphs_enabled_ = true;
    bool capturable_ = false;      // the current run so far is graph-safe
    bool capturing_ = false;
    uint64_t mem_epoch_ = 0;
    std::vector<Guard> guards_;
    std::vector<OutputRec> outs_;
    std::vector<InputSig> last_sig_;
    bool last_capturable_ = false;
    hipGraphExec_t graph_exec_ = nullptr;
    std::vector<InputSig> graph_sig_;
    std::vector<Guard> graph_guards_;
    std::vector<OutputRec> graph_outs_;
    uint64_t graph_epoch_ = 0;
};

size_t dtype_size(int dtype);

}  // namespace ortmi_ep
