// Per-fused-node plan of the MI355X EP: constants in HBM, one HIP stream, shape
// inference and kernel launches at Compute.
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "../../../include/ortmi_kernels.h"
#include "ep_internal.h"

namespace ortmi_ep {

using namespace ort_abi;

void check_hip(hipError_t e, const char* what) {
    if (e != hipSuccess) fail(std::string(what) + ": " + hipGetErrorString(e));
}

void check_kernel(int rc, const char* what) {
    if (rc != 0) fail(std::string(what) + ": " + ortmi_last_error());
}

DeviceBuffer::~DeviceBuffer() {
    if (ptr) (void)hipFree(ptr);
}

static std::unique_ptr<DeviceBuffer> device_alloc(size_t bytes) {
    auto b = std::make_unique<DeviceBuffer>();
    b->bytes = bytes;
    if (bytes) check_hip(hipMalloc(&b->ptr, bytes), "hipMalloc");
    return b;
}

// True when `p` is device memory this process can hand to a kernel.
static bool is_device_ptr(const void* p) {
    if (!p) return true;
    hipPointerAttribute_t attr;
    hipError_t e = hipPointerGetAttributes(&attr, p);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged;
}

// A fused node that is a whole int4 decoder after the decode rewrites:
//   Gather(embed, ids) -> L x [MatMulNBits q/k/v (norm prologue), GroupQueryAttention
//   (packed, in-op RoPE), MatMulNBits o_proj, MatMulNBitsSwiGLU gate/up (norm
//   prologue), MatMulNBits down] -> MatMulNBits lm_head (norm prologue) -> logits
//   [-> ArgMax over the vocabulary -> next token id].
// Its one-token steps on a device-resident KV cache shared by past and present run
// as one launch of ortmi_decoder_decode_step, the counterpart of the reference's
// one compiled-closure evaluation per token (rust/src/compiled.rs:503-822).
struct Plan::DecodeProgram {
    struct Layer {
        std::string qkv_B, qkv_S, g1, o_B, o_S, g2, gu_B, gu_S, d_B, d_S;
        float e1 = 1e-6f, e2 = 1e-6f;
        std::string past_k, past_v, present_k, present_v;
    };
    std::string ids, total, logits, embed, cos, sin, gf, lm_B, lm_S;
    std::string argmax;       // the ArgMax output, or empty when the graph has none
    bool argmax_keep = false;  // its keepdims
    bool logits_out = true;    // logits are a node output (else only the ArgMax reads them)
    float ef = 1e-6f;
    std::vector<Layer> layers;
    OrtmiDecoderDims dims{};
    std::vector<OrtmiDecoderLayer> proto;       // constant pointers resolved at Compile
    std::vector<OrtmiDecoderLayer> host_table;  // last table sent to the device
    const void *embed_p = nullptr, *cos_p = nullptr, *sin_p = nullptr, *gf_p = nullptr,
               *lm_B_p = nullptr, *lm_S_p = nullptr;
    int64_t embed_rows = 0;
    std::unique_ptr<DeviceBuffer> table, ws, next_id, logits_buf;
    size_t ws_bytes = 0;
    void* logits_ptr = nullptr;  // the last logits buffer and whether it is device memory
    bool logits_dev = false;
    void* argmax_ptr = nullptr;  // the same for the ArgMax output
    bool argmax_dev = false;
    int32_t* status = nullptr;  // host-pinned: the kernel writes it, the host reads it after the run
    // Host-pinned greedy id for an ArgMax output in host memory: the kernel writes it
    // there directly (a device-to-host copy of 8 bytes costs about 20 us per step),
    // and the host copies it to the output after the run.
    int64_t* next_host = nullptr;
    void* pending_host = nullptr;  // the host ArgMax output of the launch in flight
    int64_t steps = 0;          // program launches so far
    int64_t abort_step = 0;     // ORTMI_EP_PROGRAM_ABORT: launch to abort before it starts (1-based)
    // Plain launches until one ends with status 1 (a workgroup could not start while
    // the others waited for it); cooperative launches from then on, or always with
    // ORTMI_EP_PROGRAM_COOPERATIVE=1.
    int32_t cooperative = 0;
    ~DecodeProgram() {
        if (status) (void)hipHostFree(status);
        if (next_host) (void)hipHostFree(next_host);
    }
};

Plan::Plan(GraphIR sub, std::vector<std::string> inputs, std::vector<std::string> outputs,
           int device)
    : sub_(std::move(sub)), inputs_(std::move(inputs)), outputs_(std::move(outputs)),
      device_(device) {
    const char* fz = std::getenv("ORTMI_EP_FUSE");
    fuse_subgraph(sub_, outputs_, !(fz && std::strcmp(fz, "0") == 0));
    if (const char* g = std::getenv("ORTMI_EP_GRAPH")) graphs_enabled_ = std::strcmp(g, "0") != 0;
    check_hip(hipSetDevice(device_), "hipSetDevice");
    check_hip(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate");
    for (size_t i = 0; i < outputs_.size(); ++i)
        if (!outputs_[i].empty()) output_index_[outputs_[i]] = (int)i;
    // Past-KV inputs that only GroupQueryAttention reads are staged by its executor
    // when they arrive in host memory: with present bound to the same host buffer,
    // only the valid past rows go up and only the new rows come back.
    lazy_input_.assign(inputs_.size(), false);
    for (size_t i = 0; i < inputs_.size(); ++i) {
        if (inputs_[i].empty()) continue;
        int gqa_past = 0, other = 0;
        for (const NodeDesc& n : sub_.nodes)
            for (size_t k = 0; k < n.inputs.size(); ++k) {
                if (n.inputs[k] != inputs_[i]) continue;
                if (n.op == "GroupQueryAttention" && (k == 3 || k == 4)) ++gqa_past;
                else ++other;
            }
        lazy_input_[i] = gqa_past == 1 && other == 0;
    }
    // Constant initializers are copied to HBM once (the reference keeps a plan-owned
    // constant cache, rust/src/engine.rs:409-411).
    for (auto& kv : sub_.values) {
        ValueDesc& v = kv.second;
        if (!v.is_initializer) continue;
        auto buf = device_alloc(v.data.size());
        if (!v.data.empty())
            check_hip(hipMemcpy(buf->ptr, v.data.data(), v.data.size(), hipMemcpyHostToDevice),
                      "upload initializer");
        constants_[kv.first] = std::move(buf);
        std::vector<uint8_t>().swap(v.data);
    }
    match_decode_program();
}

void Plan::match_decode_program() {
    const auto reject = [this](const char* why) { dprog_reject_ = why; };
    const char* env = std::getenv("ORTMI_EP_PROGRAM");
    dprog_required_ = env && std::strcmp(env, "require") == 0;
    if (env && std::strcmp(env, "0") == 0) {
        dprog_reject_ = "turned off";
        return;
    }
    const auto& nodes = sub_.nodes;
    std::map<std::string, std::vector<size_t>> readers;  // value -> nodes reading it as input 0
    for (size_t i = 0; i < nodes.size(); ++i)
        if (!nodes[i].inputs.empty() && !nodes[i].inputs[0].empty()) readers[nodes[i].inputs[0]].push_back(i);
    auto in_list = [](const std::vector<std::string>& l, const std::string& v) {
        return !v.empty() && std::find(l.begin(), l.end(), v) != l.end();
    };
    auto cst = [&](const std::string& v) -> const ValueDesc* {
        auto it = sub_.values.find(v);
        return it != sub_.values.end() && it->second.is_initializer && constants_.count(v) ? &it->second
                                                                                          : nullptr;
    };
    auto reader = [&](const std::string& v, const char* op, bool norm) -> const NodeDesc* {
        auto it = readers.find(v);
        if (it == readers.end()) return nullptr;
        const NodeDesc* r = nullptr;
        for (size_t i : it->second) {
            const NodeDesc& n = nodes[i];
            if (n.op != op || (n.attr_int("__norm", 0) != 0) != norm) continue;
            if (r) return nullptr;
            r = &n;
        }
        return r;
    };
    // A 4-bit block-32 MatMulNBits with fp16 scales, no zero points, g_idx or bias.
    auto mnb = [&](const NodeDesc* n, int64_t K, int64_t N) {
        if (!n || n->attr_int("bits", 4) != 4 || n->attr_int("block_size", 32) != 32) return false;
        if (n->attr_int("K", 0) != K || (N >= 0 && n->attr_int("N", 0) != N)) return false;
        for (size_t i = 3; i < 6; ++i)
            if (n->has_input(i)) return false;
        const ValueDesc* B = cst(n->inputs[1]);
        const ValueDesc* S = cst(n->inputs[2]);
        return B && S && B->dtype == ONNX_TENSOR_ELEMENT_DATA_TYPE_UINT8 &&
               S->dtype == ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT16;
    };
    const NodeDesc* gat = nullptr;
    for (const auto& n : nodes)
        if (n.op == "Gather" && n.domain.empty()) {
            if (gat) return reject("more than one Gather");
            gat = &n;
        }
    if (!gat || gat->inputs.size() < 2 || gat->attr_int("axis", 0) != 0 || gat->outputs.empty())
        return reject("no embedding Gather");
    const ValueDesc* emb = cst(gat->inputs[0]);
    if (!emb || emb->dtype != ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT16 || emb->dims.size() != 2 ||
        !in_list(inputs_, gat->inputs[1]))
        return reject("embedding is not an fp16 [V, D] constant gathered by a node input");
    const int64_t D = emb->dims[1];
    auto dp = std::make_unique<DecodeProgram>();
    dp->ids = gat->inputs[1];
    dp->embed = gat->inputs[0];
    dprog_ids_ = dp->ids;
    std::string x = gat->outputs[0], res = x;
    int64_t H = 0, KV = 0, hd = 0, I = 0, max_pos = 0, half = 0;
    float scale = 0.f;
    for (int l = 0;; ++l) {
        const NodeDesc* q = reader(x, "MatMulNBits", true);
        if (!q || q->inputs.size() < 8 || q->outputs.empty())
            return reject("no norm prologue MatMulNBits reads the layer input");
        if (l == 0 ? q->has_input(6) : q->inputs[6] != res)
            return reject("the norm's skip input is not the residual stream");
        const NodeDesc* g = reader(q->outputs[0], "GroupQueryAttention", false);
        if (!g) {  // the lm_head: its logits are a fused-node output, an ArgMax input or both
            const NodeDesc* am = reader(q->outputs[0], "ArgMax", false);
            dp->logits_out = in_list(outputs_, q->outputs[0]);
            if (l == 0 || !(dp->logits_out || am) || !mnb(q, D, -1)) return reject("lm_head form");
            if (am) {
                auto lv = sub_.values.find(q->outputs[0]);
                const int64_t r = lv == sub_.values.end() ? 0 : (int64_t)lv->second.dims.size();
                const int64_t ax = am->attr_int("axis", 0);
                if (r != 3 || (ax != -1 && ax != 2) || am->attr_int("select_last_index", 0) != 0 ||
                    am->outputs.size() != 1 || !in_list(outputs_, am->outputs[0]))
                    return reject("ArgMax form");
                dp->argmax = am->outputs[0];
                dp->argmax_keep = am->attr_int("keepdims", 1) != 0;
            }
            dp->logits = q->outputs[0];
            dp->lm_B = q->inputs[1];
            dp->lm_S = q->inputs[2];
            dp->gf = q->inputs[7];
            dp->ef = q->attr_float("__norm_eps", 1e-6f);
            dp->dims.vocab = (int32_t)q->attr_int("N", 0);
            break;
        }
        // After layer 0 the norm before the attention adds its skip input and
        // leaves the sum (the next residual) as its output 1.
        if (l > 0) {
            if (q->outputs.size() < 2 || q->outputs[1].empty()) {
                dprog_reject_ = "the norm before the attention has no residual output";
                return;
            }
            res = q->outputs[1];
        }
        bool extra = false;  // position_ids, attention_bias, QK-norm, ...
        for (size_t i = 9; i < g->inputs.size(); ++i) extra = extra || g->has_input(i);
        if (g->inputs.size() < 9 || g->has_input(1) || g->has_input(2) ||
            g->outputs.size() < 3 || extra) {
            dprog_reject_ = "GroupQueryAttention is not the packed 9-input form";
            return;
        }
        if (g->attr_int("do_rotary", 0) != 1 || g->attr_int("rotary_interleaved", 0) != 0) {
            dprog_reject_ = "GroupQueryAttention rotary form";
            return;
        }
        if (g->attr_int("sliding_window_cache", 0)) return reject("sliding-window KV cache");
        if (!in_list(inputs_, g->inputs[3]) || !in_list(inputs_, g->inputs[4]) ||
            !in_list(outputs_, g->outputs[1]) || !in_list(outputs_, g->outputs[2]))
            return reject("KV caches are not node inputs and outputs");
        const ValueDesc* cs = cst(g->inputs[7]);
        const ValueDesc* sn = cst(g->inputs[8]);
        if (!cs || !sn || cs->dims.size() != 2 || sn->dims != cs->dims ||
            cs->dtype != ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT16)
            return reject("cos/sin caches");
        if (l == 0) {
            H = g->attr_int("num_heads", 0);
            KV = g->attr_int("kv_num_heads", 0);
            scale = g->attr_float("scale", 0.f);
            dp->total = g->inputs[6];
            dp->cos = g->inputs[7];
            dp->sin = g->inputs[8];
            max_pos = cs->dims[0];
            half = cs->dims[1];
            if (H <= 0 || KV <= 0 || q->attr_int("N", 0) % (H + 2 * KV))
                return reject("head counts");
            hd = q->attr_int("N", 0) / (H + 2 * KV);
        } else if (g->attr_int("num_heads", 0) != H || g->attr_int("kv_num_heads", 0) != KV ||
                   g->attr_float("scale", 0.f) != scale || g->inputs[6] != dp->total ||
                   g->inputs[7] != dp->cos || g->inputs[8] != dp->sin) {
            dprog_reject_ = "layers differ in attention attributes";
            return;
        }
        if (!mnb(q, D, (H + 2 * KV) * hd)) return reject("QKV projection form");
        const NodeDesc* o = reader(g->outputs[0], "MatMulNBits", false);
        if (!mnb(o, H * hd, D) || o->outputs.empty()) return reject("o_proj form");
        const NodeDesc* gu = reader(o->outputs[0], "MatMulNBitsSwiGLU", true);
        if (!gu || gu->inputs.size() < 8 || gu->inputs[6] != res || gu->outputs.size() < 2 ||
            gu->outputs[1].empty() || !mnb(gu, D, -1))
            return reject("gate/up form");
        const int64_t Il = gu->attr_int("N", 0) / 2;
        if (l == 0) I = Il;
        if (Il != I) return reject("intermediate sizes differ");
        const NodeDesc* dn = reader(gu->outputs[0], "MatMulNBits", false);
        if (!mnb(dn, I, D) || dn->outputs.empty()) return reject("down form");
        DecodeProgram::Layer L;
        L.qkv_B = q->inputs[1];
        L.qkv_S = q->inputs[2];
        L.g1 = q->inputs[7];
        L.e1 = q->attr_float("__norm_eps", 1e-6f);
        L.o_B = o->inputs[1];
        L.o_S = o->inputs[2];
        L.gu_B = gu->inputs[1];
        L.gu_S = gu->inputs[2];
        L.g2 = gu->inputs[7];
        L.e2 = gu->attr_float("__norm_eps", 1e-6f);
        L.d_B = dn->inputs[1];
        L.d_S = dn->inputs[2];
        L.past_k = g->inputs[3];
        L.past_v = g->inputs[4];
        L.present_k = g->outputs[1];
        L.present_v = g->outputs[2];
        for (const std::string* gm : {&L.g1, &L.g2}) {
            const ValueDesc* gv = cst(*gm);
            if (!gv || gv->dtype != ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT16)
                return reject("gamma dtype");
        }
        dp->layers.push_back(L);
        x = dn->outputs[0];
        res = gu->outputs[1];
    }
    // Every node of the fused node is part of the program, and it has no other outputs.
    const size_t am = dp->argmax.empty() ? 0 : 1;
    if (nodes.size() != 2 + am + 5 * dp->layers.size()) return reject("extra nodes in the fused node");
    if (outputs_.size() != (dp->logits_out ? 1 : 0) + am + 2 * dp->layers.size())
        return reject("extra outputs of the fused node");
    const ValueDesc* gf = cst(dp->gf);
    if (!gf || gf->dtype != ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT16)
        return reject("final gamma dtype");
    OrtmiDecoderDims& d = dp->dims;
    d.layers = (int32_t)dp->layers.size();
    d.hidden = (int32_t)D;
    d.num_heads = (int32_t)H;
    d.kv_num_heads = (int32_t)KV;
    d.head_size = (int32_t)hd;
    d.intermediate = (int32_t)I;
    d.max_position = (int32_t)max_pos;
    d.rotary_half = (int32_t)half;
    d.rotary_interleaved = 0;
    d.block_size = 32;
    d.dtype = ORTMI_F16;
    d.scale = scale;
    auto dev = [&](const std::string& n) { return constants_.at(n)->ptr; };
    for (const DecodeProgram::Layer& L : dp->layers) {
        OrtmiDecoderLayer t{};
        t.qkv_weight = static_cast<const uint8_t*>(dev(L.qkv_B));
        t.qkv_scales = dev(L.qkv_S);
        t.ln1_gamma = dev(L.g1);
        t.ln1_epsilon = L.e1;
        t.o_weight = static_cast<const uint8_t*>(dev(L.o_B));
        t.o_scales = dev(L.o_S);
        t.ln2_gamma = dev(L.g2);
        t.ln2_epsilon = L.e2;
        t.gate_up_weight = static_cast<const uint8_t*>(dev(L.gu_B));
        t.gate_up_scales = dev(L.gu_S);
        t.down_weight = static_cast<const uint8_t*>(dev(L.d_B));
        t.down_scales = dev(L.d_S);
        dp->proto.push_back(t);
    }
    dp->embed_p = dev(dp->embed);
    dp->embed_rows = emb->dims[0];
    dp->cos_p = dev(dp->cos);
    dp->sin_p = dev(dp->sin);
    dp->gf_p = dev(dp->gf);
    dp->lm_B_p = dev(dp->lm_B);
    dp->lm_S_p = dev(dp->lm_S);
    if (const char* ab = std::getenv("ORTMI_EP_PROGRAM_ABORT")) dp->abort_step = std::atoll(ab);
    if (const char* co = std::getenv("ORTMI_EP_PROGRAM_COOPERATIVE"))
        dp->cooperative = std::strcmp(co, "0") != 0;
    check_hip(hipHostMalloc((void**)&dp->status, sizeof(int32_t), hipHostMallocDefault),
              "hipHostMalloc");
    check_hip(hipHostMalloc((void**)&dp->next_host, sizeof(int64_t), hipHostMallocDefault),
              "hipHostMalloc");
    dp->next_id = device_alloc(sizeof(int64_t));
    dprog_ = std::move(dp);
    dprog_reject_.clear();
}

bool Plan::run_decode_program(const OrtApi* a, OrtKernelContext* ctx) {
    DecodeProgram& dp = *dprog_;
    auto skip = [&](const std::string& why) {
        if (dprog_required_) fail("decode program does not apply: " + why);
        return false;
    };
    auto ids = env_.find(dp.ids);
    if (ids == env_.end() || ids->second.numel() != 1) return false;  // a prompt step
    if (ids->second.dtype != ONNX_TENSOR_ELEMENT_DATA_TYPE_INT64) return skip("input ids not int64");
    if (!env_.count(dp.total)) return skip("no total_sequence_length");
    OrtmiDecoderDims d = dp.dims;
    std::vector<OrtmiDecoderLayer> table = dp.proto;
    int64_t cap = -1;
    for (size_t l = 0; l < dp.layers.size(); ++l) {
        const DecodeProgram::Layer& L = dp.layers[l];
        const Tensor& pk = env_.at(L.past_k);
        const Tensor& pv = env_.at(L.past_v);
        if (pk.host || pv.host || pk.dims.size() != 4 || pk.dims != pv.dims)
            return skip("the KV cache is not in device memory");
        if (pk.dims[0] != 1 || pk.dims[1] != d.kv_num_heads || pk.dims[3] != d.head_size ||
            (cap >= 0 && pk.dims[2] != cap))
            return skip("KV cache shape");
        cap = pk.dims[2];
        table[l].k_cache = pk.ptr;
        table[l].v_cache = pv.ptr;
    }
    d.kv_capacity = (int32_t)cap;
    d.cooperative = dp.cooperative;
    // A host total is checked here; one in device memory (an EP whose memory device
    // is HBM gets its inputs there) is checked by the kernel itself (status 3), which
    // saves the step a device -> host round trip.
    auto hs = host_scalars_.find(dp.total);
    if (hs != host_scalars_.end() &&
        (hs->second < 1 || hs->second > cap || hs->second > d.max_position))
        return skip("total_sequence_length out of range");
    // Present outputs must be the past buffers (KV written in place) and logits a device buffer.
    const std::vector<int64_t> pdims = {1, d.kv_num_heads, cap, d.head_size};
    for (size_t l = 0; l < dp.layers.size(); ++l) {
        if (output_buffer(dp.layers[l].present_k, pdims, a, ctx, false) != table[l].k_cache ||
            output_buffer(dp.layers[l].present_v, pdims, a, ctx, false) != table[l].v_cache)
            return skip("present is not bound to past");
    }
    void* logits = nullptr;
    if (dp.logits_out) {
        logits = output_buffer(dp.logits, {1, 1, d.vocab}, a, ctx, false);
        if (logits != dp.logits_ptr) {  // the pointer query costs microseconds: once per buffer
            dp.logits_dev = is_device_ptr(logits);
            dp.logits_ptr = logits;
        }
        if (!dp.logits_dev) return skip("logits in host memory");
    } else {  // only the ArgMax reads them: a buffer of the program's own
        if (!dp.logits_buf) dp.logits_buf = device_alloc((size_t)d.vocab * 2);
        logits = dp.logits_buf->ptr;
    }
    // The program's greedy argmax (lowest index on ties) is the ArgMax output: written
    // in place when that is device memory, else copied out after the launch.
    int64_t* next_id = static_cast<int64_t*>(dp.next_id->ptr);
    dp.pending_host = nullptr;
    if (!dp.argmax.empty()) {
        const std::vector<int64_t> od = dp.argmax_keep ? std::vector<int64_t>{1, 1, 1}
                                                       : std::vector<int64_t>{1, 1};
        void* o = output_buffer(dp.argmax, od, a, ctx, false);
        if (o != dp.argmax_ptr) {
            dp.argmax_dev = is_device_ptr(o);
            dp.argmax_ptr = o;
        }
        if (dp.argmax_dev) {
            next_id = static_cast<int64_t*>(o);
        } else {  // written by the kernel to pinned memory, copied out after the run
            next_id = dp.next_host;
            dp.pending_host = o;
        }
    }
    const size_t tb = table.size() * sizeof(OrtmiDecoderLayer);
    if (!dp.table || dp.host_table.size() != table.size() ||
        std::memcmp(dp.host_table.data(), table.data(), tb) != 0) {
        if (!dp.table) dp.table = device_alloc(tb);
        check_hip(hipMemcpyAsync(dp.table->ptr, table.data(), tb, hipMemcpyHostToDevice, stream_),
                  "decode program table");
        check_hip(hipStreamSynchronize(stream_), "decode program table");
        dp.host_table = table;
    }
    const size_t wsb = ortmi_decoder_decode_step_workspace_size(&d);
    if (!dp.ws || dp.ws_bytes < wsb) {
        dp.ws = device_alloc(wsb);
        dp.ws_bytes = wsb;
        check_hip(hipMemsetAsync(dp.ws->ptr, 0, wsb, stream_), "decode program workspace");
    }
    *dp.status = -1;
    if (++dp.steps == dp.abort_step) {
        // Diagnostic (ORTMI_EP_PROGRAM_ABORT=n): abort the n-th launch before it
        // starts, through the workspace's abort word, so the op-path fallback for a
        // step the program did not complete can be exercised. Launch index = started
        // workgroups / grid (the CU count rounded down to a multiple of 8).
        int cus = 0;
        check_hip(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device_),
                  "CU count");
        const uint64_t grid = (uint64_t)(cus - cus % 8);
        uint64_t started = 0;
        check_hip(hipMemcpyAsync(&started, dp.ws->ptr, 8, hipMemcpyDeviceToHost, stream_),
                  "abort word");
        check_hip(hipStreamSynchronize(stream_), "abort word");
        const uint32_t word = (uint32_t)(started / (grid ? grid : 1)) + 1u;
        check_hip(hipMemcpyAsync(static_cast<char*>(dp.ws->ptr) + 128, &word, 4,
                                 hipMemcpyHostToDevice, stream_),
                  "abort word");
        check_hip(hipStreamSynchronize(stream_), "abort word");
    }
    const int rc = ortmi_decoder_decode_step(
        static_cast<const OrtmiDecoderLayer*>(dp.table->ptr), &d, dp.embed_p, dp.embed_rows,
        static_cast<const int64_t*>(ids->second.ptr),
        static_cast<const int32_t*>(env_.at(dp.total).ptr), dp.cos_p, dp.sin_p, dp.gf_p, dp.ef,
        static_cast<const uint8_t*>(dp.lm_B_p), dp.lm_S_p, logits, next_id, dp.status, dp.ws->ptr,
        dp.ws_bytes, stream_);
    if (rc == ORTMI_E_INVALID) {
        const std::string why = ortmi_last_error();
        if (dprog_required_) fail("decode program rejected the decoder: " + why);
        dprog_.reset();  // this decoder's form is outside the program: op by op from now on
        dprog_reject_ = why;
        return false;
    }
    if (rc == ORTMI_E_HIP && !dprog_required_) {
        // The launch itself failed (e.g. a cooperative launch while the CUs are not
        // all free for a grid that must be co-resident): this step runs op by op.
        ++dprog_fallbacks_;
        return false;
    }
    check_kernel(rc, "decode program");
    return true;
}

Plan::~Plan() {
    if (scalar_host_) (void)hipHostFree(scalar_host_);
    if (graph_exec_) (void)hipGraphExecDestroy(graph_exec_);
    if (stream_) (void)hipStreamDestroy(stream_);
}

void* Plan::workspace(size_t bytes) {
    if (!workspace_ || workspace_->bytes < bytes) {
        if (capturing_) fail("workspace growth during graph capture");
        workspace_.reset();
        workspace_ = device_alloc(bytes);
        ++mem_epoch_;
    }
    return workspace_->ptr;
}

void* Plan::arena_alloc(size_t bytes) {
    bytes = (bytes + 255) & ~(size_t)255;
    // Chunks are kept across runs; offsets restart at every Compute.
    size_t off = arena_off_;
    size_t base = 0;
    for (auto& ch : arena_) {
        if (off < base + ch->bytes) {
            size_t local = off - base;
            if (local + bytes <= ch->bytes) {
                arena_off_ = off + bytes;
                return static_cast<char*>(ch->ptr) + local;
            }
            off = base + ch->bytes;  // skip the chunk's tail
        }
        base += ch->bytes;
    }
    if (capturing_) fail("arena growth during graph capture");
    size_t grow = std::max(bytes, (size_t)64 << 20);
    arena_.push_back(device_alloc(grow));
    ++mem_epoch_;
    arena_off_ = base + bytes;
    return arena_.back()->ptr;
}

// One-element int32 inputs in device memory (total_sequence_length, seqlens_k when
// the EP's memory device is HBM) are read back once per op-path run, in one batch:
// shapes and the graph-replay guards need their values on the host. The captured
// kernels read them from the same device buffers, so replay stays valid.
void Plan::read_device_scalars() {
    std::vector<size_t> idx;
    for (size_t i = 0; i < inputs_.size(); ++i) {
        if (inputs_[i].empty() || !devptr_[i].second || host_scalars_.count(inputs_[i])) continue;
        auto it = env_.find(inputs_[i]);
        if (it == env_.end() || it->second.dtype != ONNX_TENSOR_ELEMENT_DATA_TYPE_INT32 ||
            it->second.numel() != 1)
            continue;
        idx.push_back(i);
    }
    if (idx.empty()) return;
    if (scalar_host_n_ < idx.size()) {
        if (scalar_host_) (void)hipHostFree(scalar_host_);
        scalar_host_ = nullptr;
        check_hip(hipHostMalloc((void**)&scalar_host_, idx.size() * sizeof(int32_t),
                                hipHostMallocDefault),
                  "pinned scalars");
        scalar_host_n_ = idx.size();
    }
    for (size_t k = 0; k < idx.size(); ++k)
        check_hip(hipMemcpyAsync(scalar_host_ + k, env_.at(inputs_[idx[k]]).ptr, 4,
                                 hipMemcpyDeviceToHost, stream_),
                  "read scalar");
    check_hip(hipStreamSynchronize(stream_), "read scalar");
    for (size_t k = 0; k < idx.size(); ++k) host_scalars_[inputs_[idx[k]]] = scalar_host_[k];
}

int32_t Plan::host_i32(const std::string& name) {
    auto hs = host_scalars_.find(name);
    if (hs != host_scalars_.end()) return hs->second;
    auto it = env_.find(name);
    if (it == env_.end()) fail("missing scalar input " + name);
    int32_t v = 0;
    if (is_device_ptr(it->second.ptr)) {
        if (capturing_) fail("host read of a device scalar during graph capture");
        capturable_ = false;
        check_hip(hipMemcpyAsync(&v, it->second.ptr, 4, hipMemcpyDeviceToHost, stream_), "read scalar");
        check_hip(hipStreamSynchronize(stream_), "read scalar");
    } else {
        std::memcpy(&v, it->second.ptr, 4);
    }
    host_scalars_[name] = v;
    return v;
}

namespace {
// A device -> host copy queued for the end of a run: `height` rows of `width`
// bytes, `pitch` bytes apart on both sides (one row for a whole tensor).
struct Staged {
    void* host;
    const void* dev;
    size_t pitch, width, height;
};
thread_local std::vector<Staged>* g_out_staging = nullptr;
}  // namespace

void* Plan::output_buffer(const std::string& name, const std::vector<int64_t>& dims,
                          const OrtApi* a, OrtKernelContext* ctx, bool record) {
    auto oi = output_index_.find(name);
    if (oi == output_index_.end()) return nullptr;
    OrtValue* ov = nullptr;
    check_ort(a, api::KernelContext_GetOutput(a)(ctx, (size_t)oi->second, dims.data(), dims.size(),
                                                 &ov),
              "KernelContext_GetOutput");
    void* p = nullptr;
    check_ort(a, api::GetTensorMutableData(a)(ov, &p), "GetTensorMutableData");
    if (record) outs_.push_back({(size_t)oi->second, dims, p});
    return p;
}

void Plan::copy_out_rows(void* host, const void* dev, size_t pitch, size_t row_bytes,
                         size_t rows, size_t slabs) {
    if (capturing_) fail("host-memory output during graph capture");
    capturable_ = false;
    if (row_bytes && rows && slabs) g_out_staging->push_back({host, dev, pitch, row_bytes * rows, slabs});
}

Plan::Tensor& Plan::out_tensor(const std::string& name, int dtype,
                               const std::vector<int64_t>& dims, const OrtApi* a,
                               OrtKernelContext* ctx) {
    Tensor t;
    t.dtype = dtype;
    t.dims = dims;
    const size_t bytes = (size_t)std::max<int64_t>(t.numel(), 0) * dtype_size(dtype);
    if (output_index_.count(name)) {
        void* p = output_buffer(name, dims, a, ctx);
        if (bytes && !is_device_ptr(p)) {
            // Host-memory output: computed into the arena, copied out at the end.
            void* d = arena_alloc(bytes);
            copy_out_rows(p, d, bytes, bytes, 1, 1);
            p = d;
        }
        t.ptr = p;
    } else {
        t.ptr = bytes ? arena_alloc(bytes) : nullptr;
    }
    env_[name] = t;
    return env_[name];
}

bool Plan::guards_hold(const std::vector<Guard>& guards) const {
    for (const Guard& g : guards) {
        auto it = host_scalars_.find(g.name);
        if (it == host_scalars_.end() || it->second < 1 || it->second > g.hi) return false;
    }
    return true;
}

// Replay the captured graph when every output lands where it did at capture.
bool Plan::replay(const OrtApi* a, OrtKernelContext* ctx) {
    for (const OutputRec& o : graph_outs_) {
        OrtValue* ov = nullptr;
        check_ort(a, api::KernelContext_GetOutput(a)(ctx, o.index, o.dims.data(), o.dims.size(), &ov),
                  "KernelContext_GetOutput");
        void* p = nullptr;
        check_ort(a, api::GetTensorMutableData(a)(ov, &p), "GetTensorMutableData");
        if (p != o.ptr) return false;
    }
    check_hip(hipGraphLaunch(graph_exec_, stream_), "hipGraphLaunch");
    return true;
}

// Capture this run's launches into a graph and launch it. Returns false, with
// nothing enqueued, when some launch turns out not to be graph-safe.
bool Plan::capture(const OrtApi* a, OrtKernelContext* ctx, const std::vector<InputSig>& sig) {
    const auto saved_env = env_;
    const size_t saved_off = arena_off_;
    capturing_ = true;
    capturable_ = true;
    guards_.clear();
    outs_.clear();
    hipGraph_t graph = nullptr;
    bool ok = hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal) == hipSuccess;
    if (ok) {
        try {
            for (const NodeDesc& n : sub_.nodes) run_node(n, a, ctx);
        } catch (const std::exception&) {
            ok = false;
        }
        ok = hipStreamEndCapture(stream_, &graph) == hipSuccess && ok && capturable_;
    }
    capturing_ = false;
    hipGraphExec_t exec = nullptr;
    if (ok) ok = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) == hipSuccess;
    if (graph) (void)hipGraphDestroy(graph);
    if (!ok) {
        (void)hipGetLastError();
        env_ = saved_env;
        arena_off_ = saved_off;
        last_capturable_ = false;
        return false;
    }
    if (graph_exec_) (void)hipGraphExecDestroy(graph_exec_);
    graph_exec_ = exec;
    graph_sig_ = sig;
    graph_guards_ = guards_;
    graph_outs_ = outs_;
    graph_epoch_ = mem_epoch_;
    check_hip(hipGraphLaunch(graph_exec_, stream_), "hipGraphLaunch");
    return true;
}

void Plan::compute(const OrtApi* a, OrtKernelContext* ctx) {
    std::lock_guard<std::mutex> lock(mu_);
    check_hip(hipSetDevice(device_), "hipSetDevice");
    env_.clear();
    if (env_.bucket_count() < 2 * (inputs_.size() + sub_.values.size()))
        env_.reserve(inputs_.size() + sub_.values.size());
    host_scalars_.clear();
    arena_off_ = 0;
    std::vector<Staged> out_staging;
    g_out_staging = &out_staging;
    if (stage_.size() < inputs_.size()) stage_.resize(inputs_.size());
    if (devptr_.size() < inputs_.size()) devptr_.resize(inputs_.size(), {nullptr, false});
    if (lazy_input_.size() < inputs_.size()) lazy_input_.resize(inputs_.size(), false);
    std::vector<InputSig> sig(inputs_.size());
    for (size_t i = 0; i < inputs_.size(); ++i) {
        if (inputs_[i].empty()) continue;
        const OrtValue* v = nullptr;
        check_ort(a, api::KernelContext_GetInput(a)(ctx, i, &v), "KernelContext_GetInput");
        if (!v) continue;
        OrtTensorTypeAndShapeInfo* info = nullptr;
        check_ort(a, api::GetTensorTypeAndShape(a)(v, &info), "GetTensorTypeAndShape");
        ONNXTensorElementDataType et = ONNX_TENSOR_ELEMENT_DATA_TYPE_UNDEFINED;
        size_t nd = 0;
        OrtStatus* s1 = api::GetTensorElementType(a)(info, &et);
        OrtStatus* s2 = s1 ? nullptr : api::GetDimensionsCount(a)(info, &nd);
        Tensor t;
        t.dtype = et;
        t.dims.resize(nd);
        OrtStatus* s3 = (s1 || s2 || !nd) ? nullptr : api::GetDimensions(a)(info, t.dims.data(), nd);
        api::ReleaseTensorTypeAndShapeInfo(a)(info);
        check_ort(a, s1, "GetTensorElementType");
        check_ort(a, s2, "GetDimensionsCount");
        check_ort(a, s3, "GetDimensions");
        const void* p = nullptr;
        check_ort(a, api::GetTensorData(a)(v, &p), "GetTensorData");
        const size_t bytes = (size_t)std::max<int64_t>(t.numel(), 0) * dtype_size(et);
        if (devptr_[i].first != p || !p) devptr_[i] = {p, is_device_ptr(p)};
        sig[i].dtype = et;
        sig[i].dims = t.dims;
        if (bytes && !devptr_[i].second) {
            // Host-memory input: staged into a buffer of its own (a fixed address,
            // so graphs can read it), e.g. total_sequence_length, which ONNX
            // Runtime keeps in CPU memory.
            auto& buf = stage_[i];
            if (!buf || buf->bytes < bytes) {
                buf = device_alloc(std::max<size_t>(bytes, 256));
                ++mem_epoch_;
            }
            t.ptr = buf->ptr;
            t.host = p;
            t.lazy = lazy_input_[i];
            if (!t.lazy)
                check_hip(hipMemcpyAsync(buf->ptr, p, bytes, hipMemcpyHostToDevice, stream_),
                          "stage input");
            // keep the host copy for scalar reads without a device round trip
            if (bytes == 4 && (et == ONNX_TENSOR_ELEMENT_DATA_TYPE_INT32)) {
                int32_t hv;
                std::memcpy(&hv, p, 4);
                host_scalars_[inputs_[i]] = hv;
            }
        } else {
            t.ptr = const_cast<void*>(p);
            sig[i].ptr = p;
        }
        env_[inputs_[i]] = t;
    }
    if (!dprog_ && dprog_required_) {
        auto ids = dprog_ids_.empty() ? env_.end() : env_.find(dprog_ids_);
        if (ids == env_.end() || ids->second.numel() == 1)
            fail("decode program does not apply: " + dprog_reject_);
    }
    if (dprog_) {
        outs_.clear();
        if (run_decode_program(a, ctx)) {
            check_hip(hipStreamSynchronize(stream_), "hipStreamSynchronize");
            g_out_staging = nullptr;
            const int32_t st = *dprog_->status;
            if (st == 2) fail("decode program: input id out of range", ORT_INVALID_ARGUMENT);
            if (st == 0) {
                if (dprog_->pending_host)
                    std::memcpy(dprog_->pending_host, dprog_->next_host, sizeof(int64_t));
                return;
            }
            // Not completed (1: a wait saw no data for 100 ms; -1: the launch stopped
            // before writing a status). The step runs again op by op: the K/V row it
            // may have written at total - 1 is rewritten with the same values.
            if (dprog_required_)
                fail("decode program failed (status " + std::to_string(st) + ")");
            if (st == 1) dprog_->cooperative = 1;
            ++dprog_fallbacks_;
            outs_.clear();
        }
    }
    read_device_scalars();
    for (auto& kv : constants_) {
        const ValueDesc& v = sub_.values.at(kv.first);
        Tensor t;
        t.ptr = kv.second->ptr;
        t.dtype = v.dtype;
        t.dims = v.dims;
        env_[kv.first] = t;
    }
    if (graphs_enabled_) {
        if (graph_exec_ && graph_epoch_ != mem_epoch_) {
            (void)hipGraphExecDestroy(graph_exec_);
            graph_exec_ = nullptr;
        }
        bool done = false;
        if (graph_exec_ && sig == graph_sig_ && guards_hold(graph_guards_))
            done = replay(a, ctx);
        else if (last_capturable_ && sig == last_sig_ && guards_hold(guards_))
            done = capture(a, ctx, sig);
        if (done) {
            check_hip(hipStreamSynchronize(stream_), "hipStreamSynchronize");
            g_out_staging = nullptr;
            return;
        }
    }
    capturable_ = true;
    guards_.clear();
    outs_.clear();
    for (const NodeDesc& n : sub_.nodes) run_node(n, a, ctx);
    for (const Staged& s : out_staging)
        check_hip(hipMemcpy2DAsync(s.host, s.pitch, s.dev, s.pitch, s.width, s.height,
                                   hipMemcpyDeviceToHost, stream_),
                  "stage output");
    check_hip(hipStreamSynchronize(stream_), "hipStreamSynchronize");
    g_out_staging = nullptr;
    last_sig_ = std::move(sig);
    last_capturable_ = capturable_ && out_staging.empty();
}

// ------------------------------------------------------------ op dispatch --

static int32_t kdt(int onnx_dtype) {
    switch (onnx_dtype) {
        case ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT: return ORTMI_F32;
        case ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT16: return ORTMI_F16;
        case ONNX_TENSOR_ELEMENT_DATA_TYPE_BFLOAT16: return ORTMI_BF16;
        default: fail("unsupported element type", ORT_INVALID_ARGUMENT);
    }
}

void Plan::run_node(const NodeDesc& n, const OrtApi* a, OrtKernelContext* ctx) {
    auto in = [&](size_t i) -> Tensor* {
        if (!n.has_input(i)) return nullptr;
        auto it = env_.find(n.inputs[i]);
        if (it == env_.end()) fail(n.op + ": input " + n.inputs[i] + " is not available");
        return &it->second;
    };
    auto need = [&](size_t i) -> Tensor& {
        Tensor* t = in(i);
        if (!t) fail(n.op + ": missing input " + std::to_string(i), ORT_INVALID_ARGUMENT);
        return *t;
    };
    auto outname = [&](size_t i) -> std::string {
        return i < n.outputs.size() ? n.outputs[i] : std::string();
    };
    void* st = stream_;
    const std::string& op = n.op;

    if (op == "MatMulNBits" || op == "MatMulNBitsSwiGLU") {
        // Plain MatMulNBits, or one merged by the decode rewrites: an optional
        // (Skip)SimplifiedLayerNorm prologue (inputs 6 skip, 7 gamma; output 1 the
        // residual sum) and/or SwiGLU over interleaved gate/up rows.
        const bool pair = op == "MatMulNBitsSwiGLU";
        const bool norm = n.attr_int("__norm", 0) != 0;
        Tensor X = need(0);
        Tensor B = need(1);
        Tensor S = need(2);
        Tensor* Z = in(3);
        Tensor* skip = norm ? in(6) : nullptr;
        Tensor* gamma = norm ? &need(7) : nullptr;
        const float eps = n.attr_float("__norm_eps", 1e-6f);
        const int64_t K = n.attr_int("K", 0), N = n.attr_int("N", 0);
        const int64_t bits = n.attr_int("bits", 4), bs = n.attr_int("block_size", 32);
        if (X.dims.empty() || X.dims.back() != K) fail(op + ": A's last dim != K", ORT_INVALID_ARGUMENT);
        if (skip && skip->dims != X.dims) fail(op + ": skip shape differs", ORT_INVALID_ARGUMENT);
        const int dtype = X.dtype;
        const int64_t M = X.numel() / K;
        std::vector<int64_t> od = X.dims;
        od.back() = pair ? N / 2 : N;
        const std::string res_name = norm && n.outputs.size() > 1 ? n.outputs[1] : std::string();
        void* zp = Z ? Z->ptr : nullptr;
        if (X.splits > 0) {
            // The attention before this node left its one-token output as split
            // partials (attention-merge rewrite): merge them in the GEMV prologue.
            if (M != 1 || norm || pair) fail(op + ": split partials need a plain decode GEMV");
            Tensor& Y = out_tensor(outname(0), dtype, od, a, ctx);
            check_kernel(ortmi_matmul_nbits_decode_merge(
                             (const float*)X.ptr, X.splits, X.head, (const uint8_t*)B.ptr, S.ptr,
                             (const uint8_t*)zp, Y.ptr, N, K, bs, kdt(dtype), st),
                         op.c_str());
            return;
        }
        if (M == 1 && bits == 4 && (norm || pair) &&
            (dtype == ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT16 ||
             dtype == ONNX_TENSOR_ELEMENT_DATA_TYPE_BFLOAT16)) {
            Tensor& Y = out_tensor(outname(0), dtype, od, a, ctx);
            void* yp = Y.ptr;
            void* rp = res_name.empty() ? nullptr : out_tensor(res_name, dtype, X.dims, a, ctx).ptr;
            const int rc = ortmi_matmul_nbits_decode_fused(
                X.ptr, skip ? skip->ptr : nullptr, gamma ? gamma->ptr : nullptr, eps, rp,
                (const uint8_t*)B.ptr, S.ptr, (const uint8_t*)zp, yp, N, K, bs,
                (norm ? ORTMI_FUSE_RMS_NORM : 0) | (pair ? ORTMI_FUSE_SWIGLU_PAIRS : 0), kdt(dtype),
                st);
            if (rc == ORTMI_OK) return;
            if (rc != ORTMI_E_INVALID) check_kernel(rc, op.c_str());
        }
        // Unfused: norm into a temporary, the matmul, then SwiGLU over the pairs.
        void* ap = X.ptr;
        if (norm) {
            ap = arena_alloc((size_t)X.numel() * dtype_size(dtype));
            void* rp = res_name.empty() ? nullptr : out_tensor(res_name, dtype, X.dims, a, ctx).ptr;
            check_kernel(ortmi_rms_norm(X.ptr, skip ? skip->ptr : nullptr, nullptr, gamma->ptr, ap,
                                        rp, M, K, eps, kdt(dtype), st),
                         "SimplifiedLayerNormalization");
        }
        Tensor& Y = out_tensor(outname(0), dtype, od, a, ctx);
        if (pair && bits == 4 && M > 1 && dtype == ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT16) {
            // Prompt steps: SwiGLU in the GEMM epilogue.
            const int rc = ortmi_matmul_nbits_swiglu_pairs(ap, (const uint8_t*)B.ptr, S.ptr,
                                                           (const uint8_t*)zp, Y.ptr, M, N, K, bs,
                                                           kdt(dtype), st);
            if (rc == ORTMI_OK) return;
            if (rc != ORTMI_E_INVALID) check_kernel(rc, op.c_str());
        }
        void* yp = pair ? arena_alloc((size_t)(M * N) * dtype_size(dtype)) : Y.ptr;
        check_kernel(ortmi_matmul_nbits(ap, (const uint8_t*)B.ptr, S.ptr, (const uint8_t*)zp, yp,
                                        M, N, K, bits, bs, kdt(dtype), st),
                     "MatMulNBits");
        if (pair)
            check_kernel(ortmi_swiglu_pairs(yp, Y.ptr, M, N / 2, kdt(dtype), st), "SwiGLU");
        return;
    }
    if (op == "GroupQueryAttention") {
        Tensor q = need(0);
        Tensor* kp = in(1);
        Tensor* vp = in(2);
        Tensor* pk = in(3);
        Tensor* pv = in(4);
        if (n.attr_int("sliding_window_cache", 0)) {  // claim_gqa: past and present given
            const int64_t H = n.attr_int("num_heads", 0), KV = n.attr_int("kv_num_heads", 0);
            const int64_t B = q.dims[0], S = q.dims[1];
            const bool packed = kp == nullptr;
            const int64_t hd = packed ? q.dims[2] / (H + 2 * KV) : q.dims[2] / H;
            if (!pk || !pv || pk->dims.size() != 4 || pv->dims != pk->dims)
                fail("GroupQueryAttention: sliding cache needs past key/value of one shape",
                     ORT_INVALID_ARGUMENT);
            const int64_t cap = pk->dims[2];
            Tensor& seq = need(5);
            if (seq.numel() != B)
                fail("GroupQueryAttention: seqlens_k must have one value per batch",
                     ORT_INVALID_ARGUMENT);
            const bool rotary = n.attr_int("do_rotary", 0) != 0;
            Tensor* cs = rotary ? in(7) : nullptr;
            Tensor* sn = rotary ? in(8) : nullptr;
            if (cs && seq.host) {  // host lengths: positions checked against the cos/sin rows
                const int32_t* sl = static_cast<const int32_t*>(seq.host);
                for (int64_t b = 0; b < B; ++b)
                    if (std::max<int64_t>((int64_t)sl[b] + 1 - S, 0) + S > cs->dims[0])
                        fail("GroupQueryAttention: position exceeds the cos/sin cache",
                             ORT_INVALID_ARGUMENT);
            }
            for (Tensor* t : {pk, pv})
                if (t->lazy) {
                    check_hip(hipMemcpyAsync(t->ptr, t->host, (size_t)t->numel() * dtype_size(t->dtype),
                                             hipMemcpyHostToDevice, stream_),
                              "stage past");
                    t->lazy = false;
                }
            Tensor& O = out_tensor(outname(0), q.dtype, {B, S, H * hd}, a, ctx);
            void* optr = O.ptr;
            void* prk = out_tensor(outname(1), q.dtype, pk->dims, a, ctx).ptr;
            void* prv = out_tensor(outname(2), q.dtype, pk->dims, a, ctx).ptr;
            Tensor* qnw = in(14);
            Tensor* knw = in(15);
            const size_t wsb =
                ortmi_group_query_attention_sliding_workspace_size(B, S, H, KV, hd, cap);
            void* ws = workspace(wsb);
            check_kernel(ortmi_group_query_attention_sliding(
                             q.ptr, kp ? kp->ptr : nullptr, vp ? vp->ptr : nullptr, pk->ptr,
                             pv->ptr, cap, static_cast<const int32_t*>(seq.ptr),
                             cs ? cs->ptr : nullptr, sn ? sn->ptr : nullptr, cs ? cs->dims[1] : 0,
                             cs ? cs->dims[0] : 0, qnw ? qnw->ptr : nullptr,
                             knw ? knw->ptr : nullptr, n.attr_float("qk_norm_epsilon", 1e-6f),
                             n.attr_int("local_window_size", -1), optr, prk, prv, B, S, H, KV, hd,
                             n.attr_float("scale", 0.f), (int32_t)n.attr_int("rotary_interleaved", 0),
                             kdt(q.dtype), ws, wsb, st),
                         "GroupQueryAttention");
            return;
        }
        const int32_t total = host_i32(n.inputs[6]);
        const int64_t H = n.attr_int("num_heads", 0), KV = n.attr_int("kv_num_heads", 0);
        const int64_t B = q.dims[0], S = q.dims[1];
        const bool packed = kp == nullptr;
        const int64_t hd = packed ? q.dims[2] / (H + 2 * KV) : q.dims[2] / H;
        const int64_t cap = pk ? pk->dims[2] : 0;
        int64_t vpast = total - S;
        bool shared;
        if (vpast < 0 || vpast > cap) {
            shared = false;
            vpast = cap;
        } else {
            shared = cap > vpast;
        }
        const int64_t pcap = shared ? cap : cap + S;
        const bool rotary = n.attr_int("do_rotary", 0) != 0;
        Tensor* cs = rotary ? in(7) : nullptr;
        Tensor* sn = rotary ? in(8) : nullptr;
        void* kptr = kp ? kp->ptr : nullptr;
        void* vptr = vp ? vp->ptr : nullptr;
        void* pkp = pk ? pk->ptr : nullptr;
        void* pvp = pv ? pv->ptr : nullptr;
        void* csp = cs ? cs->ptr : nullptr;
        void* snp = sn ? sn->ptr : nullptr;
        const int64_t half = cs ? cs->dims[1] : 0, max_pos = cs ? cs->dims[0] : 0;
        Tensor& O = out_tensor(outname(0), q.dtype, {B, S, H * hd}, a, ctx);
        void* optr = O.ptr;
        void *prk = nullptr, *prv = nullptr;
        const size_t es = dtype_size(q.dtype);
        const std::vector<int64_t> pdims = {B, KV, pcap, hd};
        // Host KV shared between past and present (present bound to the past's host
        // buffer): the staging buffer is updated in place; only rows [0, valid_past)
        // go up and only the S new rows of each (batch, kv head) slab come back, as
        // the reference's delta write-back (rust/src/engine.rs:78-94, 1997-2093).
        if (shared && pk && pv && pk->host && pv->host && !outname(1).empty() &&
            !outname(2).empty()) {
            const size_t nrec = outs_.size();  // output_buffer records only fused-node outputs
            void* hk = output_buffer(outname(1), pdims, a, ctx);
            void* hv = output_buffer(outname(2), pdims, a, ctx);
            if (hk == pk->host && hv == pv->host) {
                const size_t pitch = (size_t)cap * hd * es;
                for (Tensor* t : {pk, pv}) {
                    if (t->lazy && vpast > 0)
                        check_hip(hipMemcpy2DAsync(t->ptr, pitch, t->host, pitch,
                                                   (size_t)vpast * hd * es, (size_t)(B * KV),
                                                   hipMemcpyHostToDevice, stream_),
                                  "stage past rows");
                    t->lazy = false;
                    copy_out_rows(static_cast<char*>(const_cast<void*>(t->host)) + vpast * hd * es,
                                  static_cast<char*>(t->ptr) + vpast * hd * es, pitch, hd * es,
                                  (size_t)S, (size_t)(B * KV));
                }
                prk = pk->ptr;
                prv = pv->ptr;
                pkp = prk;
                pvp = prv;
                for (int j = 1; j <= 2; ++j) {
                    Tensor t;
                    t.ptr = j == 1 ? prk : prv;
                    t.dtype = q.dtype;
                    t.dims = pdims;
                    env_[outname(j)] = t;
                }
            } else {
                // Not aliased: drop the records just made; out_tensor below fetches
                // the outputs again and stages them whole.
                outs_.resize(nrec);
            }
        }
        for (Tensor* t : {pk, pv})
            if (t && t->lazy) {  // any other host past: the whole buffer goes up
                check_hip(hipMemcpyAsync(t->ptr, t->host, (size_t)t->numel() * es,
                                         hipMemcpyHostToDevice, stream_),
                          "stage past");
                t->lazy = false;
            }
        if (!prk) {
            if (!outname(1).empty()) prk = out_tensor(outname(1), q.dtype, pdims, a, ctx).ptr;
            else prk = arena_alloc((size_t)(B * KV * pcap * hd) * es);
            if (!outname(2).empty()) prv = out_tensor(outname(2), q.dtype, pdims, a, ctx).ptr;
            else prv = arena_alloc((size_t)(B * KV * pcap * hd) * es);
        }
        const float scale = n.attr_float("scale", 0.f);
        const int32_t inter = (int32_t)n.attr_int("rotary_interleaved", 0);
        // fp32, attention_bias, QK-norm and head sizes other than 64/96/128 run the
        // generic kernels (one prep launch, one attention launch).
        Tensor* bias = in(10);
        Tensor* qnw = in(14);
        Tensor* knw = in(15);
        if (q.dtype == ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT || bias || qnw || knw ||
            (hd != 64 && hd != 96 && hd != 128)) {
            if (capturing_) fail("GroupQueryAttention form is not capturable");
            capturable_ = false;
            int64_t bd[4] = {0, 0, 0, 0};
            if (bias) {
                if (bias->dims.size() != 4)
                    fail("GroupQueryAttention: attention_bias must be rank 4");
                for (int i = 0; i < 4; ++i) bd[i] = bias->dims[i];
            }
            const size_t wsb = ortmi_group_query_attention_ex_workspace_size(B, S, H, hd);
            void* ws = workspace(wsb);
            check_kernel(ortmi_group_query_attention_ex(
                             q.ptr, kptr, vptr, pkp, pvp, cap, total, csp, snp, half, max_pos,
                             qnw ? qnw->ptr : nullptr, knw ? knw->ptr : nullptr,
                             n.attr_float("qk_norm_epsilon", 1e-6f), bias ? bias->ptr : nullptr,
                             bd[0], bd[1], bd[2], bd[3], optr, prk, prv, B, S, H, KV, hd, scale,
                             inter, kdt(q.dtype), ws, wsb, st),
                         "GroupQueryAttention");
            return;
        }
        // One-token decode into a shared buffer written in place: the capturable
        // kernels read total_sequence_length from device memory, so the step can
        // be replayed from a graph. Eager runs take the same kernels, so replayed
        // and eager steps give identical results.
        if (S == 1 && shared && pk && pv && prk == pkp && prv == pvp &&
            host_scalars_.count(n.inputs[6]) && (!cs || total <= max_pos)) {
            const int32_t* tdev = (const int32_t*)env_.at(n.inputs[6]).ptr;
            // Partials for the o_proj GEMV to merge, unless their bound (the GEMV
            // stages all heads' partials) leaves too few key splits: with 32 heads of
            // 128 one split walks the whole context in one workgroup per KV head
            // (Mistral-7B's layout at 640 keys: 11.8 us per layer against 4 us split).
            const int64_t nsp = ortmi_group_query_attention_decode_splits(B, H, KV, hd, cap);
            if (B == 1 && n.attr_int("__partials", 0) && nsp > 0 &&
                nsp >= std::min<int64_t>(4, (cap + 255) / 256)) {
                // Output left as split partials for the o_proj GEMV to merge.
                const int64_t ns = nsp;
                float* part = (float*)arena_alloc((size_t)(B * H * ns * (hd + 2)) * sizeof(float));
                const int rc = ortmi_group_query_attention_decode_partials(
                    q.ptr, kptr, vptr, prk, prv, cap, tdev, csp, snp, half, max_pos, part, B, H,
                    KV, hd, scale, inter, kdt(q.dtype), st);
                if (rc == ORTMI_OK) {
                    Tensor& o = env_[outname(0)];
                    o.ptr = part;
                    o.splits = ns;
                    o.head = hd;
                    guards_.push_back({n.inputs[6], cs ? std::min<int64_t>(cap, max_pos) : cap});
                    return;
                }
                if (rc != ORTMI_E_INVALID) check_kernel(rc, "GroupQueryAttention");
            }
            const size_t wsb = ortmi_group_query_attention_workspace_size(B, 1, H, hd, cap);
            void* ws = workspace(wsb);
            const int rc = ortmi_group_query_attention_decode_capturable(
                q.ptr, kptr, vptr, prk, prv, cap, tdev, csp, snp, half, max_pos, optr, B, H, KV,
                hd, scale, inter, kdt(q.dtype), ws, wsb, st);
            if (rc == ORTMI_OK) {
                guards_.push_back({n.inputs[6], cs ? std::min<int64_t>(cap, max_pos) : cap});
                return;
            }
            if (rc != ORTMI_E_INVALID) check_kernel(rc, "GroupQueryAttention");
        }
        if (capturing_) fail("GroupQueryAttention form is not capturable");
        capturable_ = false;
        const size_t wsb = ortmi_group_query_attention_workspace_size(B, S, H, hd, vpast + S);
        void* ws = workspace(wsb);
        check_kernel(ortmi_group_query_attention(q.ptr, kptr, vptr, pkp, pvp, cap, total, csp, snp,
                                                 half, max_pos, optr, prk, prv, B, S, H, KV, hd,
                                                 scale, inter, kdt(q.dtype), ws, wsb, st),
                     "GroupQueryAttention");
        return;
    }
    if (op == "PagedAttention") {
        if (capturing_) fail("PagedAttention is not captured");
        capturable_ = false;
        Tensor q = need(0);
        Tensor k = need(1);
        Tensor* v = in(2);
        Tensor kc = need(3);
        Tensor* vc = in(4);
        Tensor cum = need(5), past = need(6), bt = need(7);
        const bool latent = n.attr_str("kv_cache_layout", "SEPARATE") == "LATENT";
        const bool rotary = n.attr_int("do_rotary", 0) != 0;
        Tensor* cs = rotary ? in(8) : nullptr;
        Tensor* sn = rotary ? in(9) : nullptr;
        Tensor* sm = in(10);
        Tensor* sink = in(11);
        Tensor* qw = in(12);
        Tensor* kw = in(13);
        const int64_t H = n.attr_int("num_heads", 0), KV = n.attr_int("kv_num_heads", 0);
        const int64_t T = q.dims[0], nblk = kc.dims[0], blk = kc.dims[1], hd = kc.dims[3];
        const int64_t vhd = n.attr_int("v_head_size", 0) ? n.attr_int("v_head_size", 0) : hd;
        const int64_t batch = cum.dims[0] - 1, maxb = bt.dims.size() == 2 ? bt.dims[1] : 0;
        const int64_t max_ctx = maxb * blk;
        Tensor& O = out_tensor(outname(0), q.dtype, {T, H * vhd}, a, ctx);
        const size_t wsb = ortmi_paged_attention_workspace_size(T, batch, H, KV, hd, vhd, max_ctx);
        workspace(wsb);
        check_kernel(ortmi_paged_attention(
                         q.ptr, k.ptr, latent ? nullptr : (v ? v->ptr : nullptr), kc.ptr,
                         latent ? nullptr : (vc ? vc->ptr : nullptr), nblk, blk,
                         (const int32_t*)cum.ptr, (const int32_t*)past.ptr, (const int32_t*)bt.ptr,
                         batch, maxb, T, max_ctx, cs ? cs->ptr : nullptr, sn ? sn->ptr : nullptr,
                         cs ? cs->dims[1] : 0, cs ? cs->dims[0] : 0,
                         (int32_t)n.attr_int("rotary_interleaved", 0), n.attr_int("rotary_offset", 0),
                         sm ? (const int32_t*)sm->ptr : nullptr, sink ? sink->ptr : nullptr,
                         qw ? qw->ptr : nullptr, kw ? kw->ptr : nullptr,
                         n.attr_float("qk_norm_epsilon", 1e-6f), O.ptr, H, KV, hd, vhd,
                         n.attr_float("scale", 0.f), kdt(q.dtype), workspace_->ptr,
                         workspace_->bytes, st),
                     "PagedAttention");
        // Updated caches: written in place (rust/src/engine.rs:823-847,
        // rust/src/ops/attention.rs:2728-2742). A cache that arrived in host memory
        // was updated in its device staging copy, which goes back to the caller's
        // buffer after the run. Outputs 1/2, when requested, receive the same
        // contents.
        const Tensor* caches[2] = {&kc, vc};
        for (int i = 0; i < 2; ++i) {
            if (caches[i] && caches[i]->host) {
                const size_t bytes = (size_t)caches[i]->numel() * dtype_size(caches[i]->dtype);
                copy_out_rows(const_cast<void*>(caches[i]->host), caches[i]->ptr, bytes, bytes,
                              1, 1);
            }
        }
        for (int i = 0; i < 2; ++i) {
            if (outname(1 + i).empty() || !caches[i]) continue;
            Tensor& oc = out_tensor(outname(1 + i), caches[i]->dtype, caches[i]->dims, a, ctx);
            if (oc.ptr != caches[i]->ptr)
                check_hip(hipMemcpyAsync(oc.ptr, caches[i]->ptr,
                                         (size_t)caches[i]->numel() * dtype_size(caches[i]->dtype),
                                         hipMemcpyDeviceToDevice, stream_),
                          "cache output");
        }
        return;
    }
    if (op == "RotaryEmbedding") {
        const bool ms = n.domain == "com.microsoft";
        Tensor x = need(0);
        Tensor* pos = ms ? in(1) : in(3);
        Tensor cs = need(ms ? 2 : 1), sn = need(ms ? 3 : 2);
        const bool bnsd = x.dims.size() == 4;
        int64_t B, S, NH, hd;
        if (bnsd) {
            B = x.dims[0];
            NH = x.dims[1];
            S = x.dims[2];
            hd = x.dims[3];
        } else {
            B = x.dims[0];
            S = x.dims[1];
            const int64_t nh_attr = n.attr_int("num_heads", 0);
            hd = nh_attr > 0 ? x.dims[2] / nh_attr : 2 * cs.dims.back();
            NH = x.dims[2] / hd;
        }
        // The cache's last dim is the rotated half width (rust/src/ops/attention.rs:
        // 1234-1282): dims from 2 * half on keep their values.
        const int64_t half = cs.dims.back();
        const int64_t rows = cs.numel() / half;
        Tensor& Y = out_tensor(outname(0), x.dtype, x.dims, a, ctx);
        check_kernel(ortmi_rotary_embedding(x.ptr, pos ? (const int64_t*)pos->ptr : nullptr,
                                            pos && pos->numel() == 1 ? 1 : 0, cs.ptr, sn.ptr, rows,
                                            Y.ptr, B, S, NH, hd, half, bnsd ? 1 : 0,
                                            (int32_t)n.attr_int("interleaved", 0), kdt(x.dtype), st),
                     "RotaryEmbedding");
        return;
    }
    if (op == "SimplifiedLayerNormalization" || op == "RMSNormalization" ||
        op == "SkipSimplifiedLayerNormalization") {
        const bool skip = op == "SkipSimplifiedLayerNormalization";
        Tensor x = need(0);
        Tensor* sk = skip ? &need(1) : nullptr;
        Tensor& g = need(skip ? 2 : 1);
        Tensor* bias = skip ? in(3) : nullptr;
        const int64_t D = x.dims.back();
        const float eps = n.attr_float("epsilon", skip ? 1e-6f : 1e-5f);
        void* skp = sk ? sk->ptr : nullptr;
        void* gp = g.ptr;
        void* bp = bias ? bias->ptr : nullptr;
        Tensor& Y = out_tensor(outname(0), x.dtype, x.dims, a, ctx);
        void* yp = Y.ptr;
        void* rp = nullptr;
        // input_skip_bias_sum is output 3 (outputs 1 and 2, mean and inv_std_var,
        // are declared-but-unread when the node is claimed).
        if (skip && n.outputs.size() >= 4 && !n.outputs[3].empty())
            rp = out_tensor(n.outputs[3], x.dtype, x.dims, a, ctx).ptr;
        check_kernel(ortmi_rms_norm(x.ptr, skp, bp, gp, yp, rp, x.numel() / D, D, eps,
                                    kdt(x.dtype), st),
                     op.c_str());
        return;
    }
    if (op == "Add" || op == "Mul" || op == "Sub") {
        Tensor x = need(0), y = need(1);
        if (x.dims != y.dims) fail(op + ": runtime shapes differ", ORT_INVALID_ARGUMENT);
        Tensor& O = out_tensor(outname(0), x.dtype, x.dims, a, ctx);
        check_kernel(ortmi_binary(op == "Add" ? 0 : (op == "Mul" ? 1 : 2), x.ptr, y.ptr, O.ptr,
                                  x.numel(), kdt(x.dtype), st),
                     op.c_str());
        return;
    }
    if (op == "Sigmoid") {
        Tensor x = need(0);
        Tensor& O = out_tensor(outname(0), x.dtype, x.dims, a, ctx);
        check_kernel(ortmi_sigmoid(x.ptr, O.ptr, x.numel(), kdt(x.dtype), st), "Sigmoid");
        return;
    }
    if (op == "SwiGLU") {  // fused Sigmoid -> Mul -> Mul (fuse_swiglu)
        Tensor g = need(0), u = need(1);
        if (g.dims != u.dims) fail("SwiGLU: gate and up shapes differ", ORT_INVALID_ARGUMENT);
        Tensor& O = out_tensor(outname(0), g.dtype, g.dims, a, ctx);
        check_kernel(ortmi_swiglu(g.ptr, u.ptr, O.ptr, g.numel(), kdt(g.dtype), st), "SwiGLU");
        return;
    }
    if (op == "Cast") {
        Tensor x = need(0);
        const int to = (int)n.attr_int("to", 0);
        Tensor& O = out_tensor(outname(0), to, x.dims, a, ctx);
        check_kernel(ortmi_cast(x.ptr, kdt(x.dtype), O.ptr, kdt(to), x.numel(), st), "Cast");
        return;
    }
    if (op == "Gather") {
        Tensor tab = need(0), ids = need(1);
        std::vector<int64_t> od = ids.dims;
        od.push_back(tab.dims[1]);
        Tensor& O = out_tensor(outname(0), tab.dtype, od, a, ctx);
        check_kernel(ortmi_gather_rows(tab.ptr, (const int64_t*)ids.ptr, O.ptr, ids.numel(),
                                       tab.dims[0], tab.dims[1], kdt(tab.dtype), st),
                     "Gather");
        return;
    }
    if (op == "ArgMax") {  // any axis, either tie rule (claim_argmax)
        Tensor x = need(0);
        const int64_t r = (int64_t)x.dims.size();
        if (r == 0) fail("ArgMax: scalar input", ORT_INVALID_ARGUMENT);
        int64_t axis = n.attr_int("axis", 0);
        if (axis < 0) axis += r;
        if (axis < 0 || axis >= r) fail("ArgMax: axis out of range", ORT_INVALID_ARGUMENT);
        const int64_t dim = x.dims[axis];
        if (dim <= 0) fail("ArgMax: the reduced axis is empty", ORT_INVALID_ARGUMENT);
        int64_t outer = 1, inner = 1;
        for (int64_t i = 0; i < axis; ++i) outer *= x.dims[i];
        for (int64_t i = axis + 1; i < r; ++i) inner *= x.dims[i];
        const bool last = n.attr_int("select_last_index", 0) != 0;
        std::vector<int64_t> od;
        for (int64_t i = 0; i < r; ++i)
            if (i != axis) od.push_back(x.dims[i]);
            else if (n.attr_int("keepdims", 1)) od.push_back(1);
        Tensor& O = out_tensor(outname(0), ONNX_TENSOR_ELEMENT_DATA_TYPE_INT64, od, a, ctx);
        if (outer * inner == 0) return;
        if (inner == 1 && !last && outer <= 65535) {  // greedy decoding: two passes per row
            const size_t wsb = ortmi_argmax_rows_workspace_size(outer, dim);
            void* ws = wsb ? workspace(wsb) : nullptr;
            check_kernel(ortmi_argmax_rows(x.ptr, (int64_t*)O.ptr, outer, dim, kdt(x.dtype), ws,
                                           wsb, st),
                         "ArgMax");
        } else {
            check_kernel(ortmi_argmax_axis(x.ptr, (int64_t*)O.ptr, outer, dim, inner, last ? 1 : 0,
                                           kdt(x.dtype), st),
                         "ArgMax");
        }
        return;
    }
    if (op == "GatherBlockQuantized") {
        Tensor data = need(0), ids = need(1), sc = need(2);
        Tensor* zp = in(3);
        if (data.dims.size() != 2) fail(op + ": data must be rank 2", ORT_INVALID_ARGUMENT);
        const int64_t V = data.dims[0], D = data.dims[1] * 2;
        const int64_t block = n.attr_int("block_size", 128);
        if (sc.numel() != V * ((D + block - 1) / block))
            fail(op + ": scales must be [V, ceil(D/block_size)]", ORT_INVALID_ARGUMENT);
        std::vector<int64_t> od = ids.dims;
        od.push_back(D);
        Tensor& O = out_tensor(outname(0), sc.dtype, od, a, ctx);
        check_kernel(ortmi_gather_block_quantized(
                         (const uint8_t*)data.ptr, sc.ptr, zp ? (const uint8_t*)zp->ptr : nullptr,
                         ids.ptr, ids.dtype == ONNX_TENSOR_ELEMENT_DATA_TYPE_INT64 ? 1 : 0, O.ptr,
                         ids.numel(), V, D, block, n.attr_int("bits", 4), kdt(sc.dtype), st),
                     op.c_str());
        return;
    }
    fail("no executor for " + op, ORT_NOT_IMPLEMENTED);
}

}  // namespace ortmi_ep
