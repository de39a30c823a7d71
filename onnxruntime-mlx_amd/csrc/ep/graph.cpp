// Graph reading, claim predicates and convex clustering for the MI355X EP.
#include <algorithm>
#include <cstring>
#include <functional>
#include <sstream>

#include "ep_internal.h"

namespace ortmi_ep {

using namespace ort_abi;

void check_ort(const OrtApi* a, OrtStatus* st, const char* what) {
    if (!st) return;
    std::string msg = std::string(what) + ": " + api::GetErrorMessage(a)(st);
    OrtErrorCode code = api::GetErrorCode(a)(st);
    api::ReleaseStatus(a)(st);
    throw EpError(code == ORT_OK ? ORT_EP_FAIL : code, msg);
}

size_t dtype_size(int dt) {
    switch (dt) {
        case ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT:
        case ONNX_TENSOR_ELEMENT_DATA_TYPE_INT32:
        case ONNX_TENSOR_ELEMENT_DATA_TYPE_UINT32: return 4;
        case ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT16:
        case ONNX_TENSOR_ELEMENT_DATA_TYPE_BFLOAT16:
        case ONNX_TENSOR_ELEMENT_DATA_TYPE_INT16:
        case ONNX_TENSOR_ELEMENT_DATA_TYPE_UINT16: return 2;
        case ONNX_TENSOR_ELEMENT_DATA_TYPE_INT64:
        case ONNX_TENSOR_ELEMENT_DATA_TYPE_UINT64:
        case ONNX_TENSOR_ELEMENT_DATA_TYPE_DOUBLE: return 8;
        case ONNX_TENSOR_ELEMENT_DATA_TYPE_UINT8:
        case ONNX_TENSOR_ELEMENT_DATA_TYPE_INT8:
        case ONNX_TENSOR_ELEMENT_DATA_TYPE_BOOL: return 1;
        default: return 0;
    }
}

// --------------------------------------------------------------- reading --

static void read_value_info(const OrtApi* a, const OrtValueInfo* vi, GraphIR& g,
                            std::string* name_out) {
    const char* name = nullptr;
    check_ort(a, api::GetValueInfoName(a)(vi, &name), "GetValueInfoName");
    std::string nm = name ? name : "";
    if (name_out) *name_out = nm;
    if (g.values.count(nm)) return;
    ValueDesc v;
    v.name = nm;
    const OrtTypeInfo* ti = nullptr;
    check_ort(a, api::GetValueInfoTypeInfo(a)(vi, &ti), "GetValueInfoTypeInfo");
    if (ti) {
        ONNXType ot = ONNX_TYPE_UNKNOWN;
        check_ort(a, api::GetOnnxTypeFromTypeInfo(a)(ti, &ot), "GetOnnxTypeFromTypeInfo");
        if (ot == ONNX_TYPE_TENSOR) {
            const OrtTensorTypeAndShapeInfo* tsi = nullptr;
            check_ort(a, api::CastTypeInfoToTensorInfo(a)(ti, &tsi), "CastTypeInfoToTensorInfo");
            if (tsi) {
                ONNXTensorElementDataType et = ONNX_TENSOR_ELEMENT_DATA_TYPE_UNDEFINED;
                check_ort(a, api::GetTensorElementType(a)(tsi, &et), "GetTensorElementType");
                v.dtype = et;
                size_t nd = 0;
                check_ort(a, api::GetDimensionsCount(a)(tsi, &nd), "GetDimensionsCount");
                v.dims.resize(nd);
                if (nd) check_ort(a, api::GetDimensions(a)(tsi, v.dims.data(), nd), "GetDimensions");
                v.has_shape = true;
            }
        }
    }
    bool is_const = false;
    check_ort(a, api::ValueInfo_IsConstantInitializer(a)(vi, &is_const),
              "ValueInfo_IsConstantInitializer");
    if (is_const) {
        const OrtValue* val = nullptr;
        check_ort(a, api::ValueInfo_GetInitializerValue(a)(vi, &val),
                  "ValueInfo_GetInitializerValue");
        if (val) {
            OrtTensorTypeAndShapeInfo* tsi = nullptr;
            check_ort(a, api::GetTensorTypeAndShape(a)(val, &tsi), "GetTensorTypeAndShape");
            size_t count = 0;
            ONNXTensorElementDataType et = ONNX_TENSOR_ELEMENT_DATA_TYPE_UNDEFINED;
            size_t nd = 0;
            OrtStatus* s1 = api::GetTensorShapeElementCount(a)(tsi, &count);
            OrtStatus* s2 = s1 ? nullptr : api::GetTensorElementType(a)(tsi, &et);
            OrtStatus* s3 = (s1 || s2) ? nullptr : api::GetDimensionsCount(a)(tsi, &nd);
            std::vector<int64_t> dims(nd);
            OrtStatus* s4 = (s1 || s2 || s3 || !nd) ? nullptr
                                                   : api::GetDimensions(a)(tsi, dims.data(), nd);
            api::ReleaseTensorTypeAndShapeInfo(a)(tsi);
            check_ort(a, s1, "GetTensorShapeElementCount");
            check_ort(a, s2, "GetTensorElementType");
            check_ort(a, s3, "GetDimensionsCount");
            check_ort(a, s4, "GetDimensions");
            const void* data = nullptr;
            check_ort(a, api::GetTensorData(a)(val, &data), "GetTensorData");
            const size_t bytes = count * dtype_size(et);
            v.dtype = et;
            v.dims = dims;
            v.has_shape = true;
            v.is_initializer = true;
            // Initializer bytes are copied: graph pointers do not outlive Compile
            // (rust/src/ep.rs:1003-1008, 1270-1298).
            v.data.resize(bytes);
            if (bytes && data) std::memcpy(v.data.data(), data, bytes);
        }
    }
    g.values.emplace(nm, std::move(v));
}

static void read_attr(const OrtApi* a, const OrtOpAttr* at, NodeDesc& n) {
    const char* name = nullptr;
    check_ort(a, api::OpAttr_GetName(a)(at, &name), "OpAttr_GetName");
    OrtOpAttrType t = ORT_OP_ATTR_UNDEFINED;
    check_ort(a, api::OpAttr_GetType(a)(at, &t), "OpAttr_GetType");
    Attr v;
    v.type = t;
    size_t out = 0;
    auto read_buf = [&](std::vector<uint8_t>& buf) {
        buf.resize(256);
        OrtStatus* st = api::ReadOpAttr(a)(at, t, buf.data(), buf.size(), &out);
        if (st) {  // buffer too small: `out` holds the size needed
            api::ReleaseStatus(a)(st);
            buf.resize(out);
            check_ort(a, api::ReadOpAttr(a)(at, t, buf.data(), buf.size(), &out), "ReadOpAttr");
        }
        buf.resize(out);
    };
    switch (t) {
        case ORT_OP_ATTR_INT:
            check_ort(a, api::ReadOpAttr(a)(at, t, &v.i, sizeof(v.i), &out), "ReadOpAttr");
            v.f = (float)v.i;
            break;
        case ORT_OP_ATTR_FLOAT:
            check_ort(a, api::ReadOpAttr(a)(at, t, &v.f, sizeof(v.f), &out), "ReadOpAttr");
            break;
        case ORT_OP_ATTR_STRING: {
            std::vector<uint8_t> buf;
            read_buf(buf);
            v.s.assign(buf.begin(), buf.end());
            while (!v.s.empty() && v.s.back() == '\0') v.s.pop_back();
            break;
        }
        case ORT_OP_ATTR_INTS: {
            std::vector<uint8_t> buf;
            read_buf(buf);
            v.ints.resize(buf.size() / sizeof(int64_t));
            if (!v.ints.empty()) std::memcpy(v.ints.data(), buf.data(), v.ints.size() * 8);
            break;
        }
        case ORT_OP_ATTR_FLOATS: {
            std::vector<uint8_t> buf;
            read_buf(buf);
            v.floats.resize(buf.size() / sizeof(float));
            if (!v.floats.empty()) std::memcpy(v.floats.data(), buf.data(), v.floats.size() * 4);
            break;
        }
        default:
            break;  // graph / tensor attributes are not used by claimed ops
    }
    n.attrs[name ? name : ""] = std::move(v);
}

GraphIR read_graph(const OrtApi* a, const OrtGraph* graph) {
    GraphIR g;
    auto read_list = [&](auto count_fn, auto get_fn, std::vector<std::string>& names,
                         const char* what) {
        size_t n = 0;
        check_ort(a, count_fn(a)(graph, &n), what);
        std::vector<const OrtValueInfo*> vis(n);
        if (n) check_ort(a, get_fn(a)(graph, vis.data(), n), what);
        for (auto* vi : vis) {
            std::string nm;
            if (vi) read_value_info(a, vi, g, &nm);
            names.push_back(nm);
        }
    };
    read_list(api::Graph_GetNumInputs, api::Graph_GetInputs, g.inputs, "Graph_GetInputs");
    read_list(api::Graph_GetNumOutputs, api::Graph_GetOutputs, g.outputs, "Graph_GetOutputs");
    std::vector<std::string> inits;
    read_list(api::Graph_GetNumInitializers, api::Graph_GetInitializers, inits,
              "Graph_GetInitializers");

    size_t nn = 0;
    check_ort(a, api::Graph_GetNumNodes(a)(graph, &nn), "Graph_GetNumNodes");
    std::vector<const OrtNode*> nodes(nn);
    if (nn) check_ort(a, api::Graph_GetNodes(a)(graph, nodes.data(), nn), "Graph_GetNodes");
    for (const OrtNode* node : nodes) {
        NodeDesc n;
        n.handle = node;
        const char* s = nullptr;
        check_ort(a, api::Node_GetOperatorType(a)(node, &s), "Node_GetOperatorType");
        n.op = s ? s : "";
        check_ort(a, api::Node_GetDomain(a)(node, &s), "Node_GetDomain");
        n.domain = s ? s : "";
        if (n.domain == "ai.onnx") n.domain = "";
        check_ort(a, api::Node_GetName(a)(node, &s), "Node_GetName");
        n.name = s ? s : "";
        check_ort(a, api::Node_GetId(a)(node, &n.id), "Node_GetId");
        check_ort(a, api::Node_GetSinceVersion(a)(node, &n.since_version), "Node_GetSinceVersion");
        size_t ni = 0, no = 0, na = 0;
        check_ort(a, api::Node_GetNumInputs(a)(node, &ni), "Node_GetNumInputs");
        std::vector<const OrtValueInfo*> ins(ni);
        if (ni) check_ort(a, api::Node_GetInputs(a)(node, ins.data(), ni), "Node_GetInputs");
        for (auto* vi : ins) {
            std::string nm;
            if (vi) read_value_info(a, vi, g, &nm);
            n.inputs.push_back(nm);
        }
        check_ort(a, api::Node_GetNumOutputs(a)(node, &no), "Node_GetNumOutputs");
        std::vector<const OrtValueInfo*> outs(no);
        if (no) check_ort(a, api::Node_GetOutputs(a)(node, outs.data(), no), "Node_GetOutputs");
        for (auto* vi : outs) {
            std::string nm;
            if (vi) read_value_info(a, vi, g, &nm);
            n.outputs.push_back(nm);
        }
        check_ort(a, api::Node_GetNumAttributes(a)(node, &na), "Node_GetNumAttributes");
        std::vector<const OrtOpAttr*> attrs(na);
        if (na) check_ort(a, api::Node_GetAttributes(a)(node, attrs.data(), na), "Node_GetAttributes");
        for (auto* at : attrs)
            if (at) read_attr(a, at, n);
        g.nodes.push_back(std::move(n));
    }
    return g;
}

// ------------------------------------------------------------------ claims --

namespace {

const ValueDesc* val(const GraphIR& g, const NodeDesc& n, size_t i) {
    if (!n.has_input(i)) return nullptr;
    auto it = g.values.find(n.inputs[i]);
    return it == g.values.end() ? nullptr : &it->second;
}
const ValueDesc* out_val(const GraphIR& g, const NodeDesc& n, size_t i) {
    if (i >= n.outputs.size() || n.outputs[i].empty()) return nullptr;
    auto it = g.values.find(n.outputs[i]);
    return it == g.values.end() ? nullptr : &it->second;
}
bool is_float(int dt) {
    return dt == ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT || dt == ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT16 ||
           dt == ONNX_TENSOR_ELEMENT_DATA_TYPE_BFLOAT16;
}
bool is_half(int dt) {
    return dt == ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT16 || dt == ONNX_TENSOR_ELEMENT_DATA_TYPE_BFLOAT16;
}
std::string fmt(const char* s) { return s; }
std::string fmt(const std::string& s) { return s; }

#define REQUIRE(cond, msg) \
    do {                   \
        if (!(cond)) return fmt(msg); \
    } while (0)

// rust/src/ops/quant.rs:1655-1711
std::string claim_matmulnbits(const NodeDesc& n, const GraphIR& g) {
    REQUIRE(!n.outputs.empty() && !n.outputs[0].empty(), "requires at least one output");
    auto* out = out_val(g, n, 0);
    auto *a = val(g, n, 0), *b = val(g, n, 1), *s = val(g, n, 2);
    REQUIRE(out && a && b && s, "missing tensor type/shape info on an input");
    REQUIRE(is_float(out->dtype), "output must be a float (fp32/fp16/bf16)");
    REQUIRE(is_float(a->dtype) && b->dtype == ONNX_TENSOR_ELEMENT_DATA_TYPE_UINT8 &&
                is_float(s->dtype),
            "activation/scales must be float and packed weights uint8");
    REQUIRE(a->dtype == s->dtype && a->dtype == out->dtype,
            "activation, scales and output must share one float dtype");
    if (n.has_input(3)) {
        auto* zp = val(g, n, 3);
        REQUIRE(zp && zp->dtype == ONNX_TENSOR_ELEMENT_DATA_TYPE_UINT8,
                "zero_points must be uint8 when present");
    }
    for (size_t i = 4; i < n.inputs.size(); ++i)
        REQUIRE(!n.has_input(i), "g_idx and bias inputs are not supported");
    const int64_t bits = n.attr_int("bits", 4), block = n.attr_int("block_size", 32);
    REQUIRE(bits == 4 || bits == 8, "only 4-bit and 8-bit weights are supported");
    REQUIRE(block == 16 || block == 32 || block == 64 || block == 128,
            "block_size must be 16, 32, 64, or 128");
    REQUIRE(n.attr_int("K", 0) > 0 && n.attr_int("N", 0) > 0, "missing K/N");
    return "";
}

// rust/src/ops/attention.rs:1527-1738, restricted to what the gfx950 kernels run.
std::string claim_gqa(const NodeDesc& n, const GraphIR& g) {
    REQUIRE(n.inputs.size() >= 7 && n.inputs.size() <= 16, "GroupQueryAttention needs 7-16 inputs");
    REQUIRE(!n.outputs.empty() && !n.outputs[0].empty(), "GroupQueryAttention needs an output");
    const int64_t H = n.attr_int("num_heads", 0), KV = n.attr_int("kv_num_heads", 0);
    REQUIRE(H > 0 && KV > 0 && H % KV == 0, "num_heads must be a multiple of kv_num_heads");
    auto* q = val(g, n, 0);
    REQUIRE(q && q->has_shape && q->dims.size() == 3, "query must be rank 3");
    REQUIRE(is_float(q->dtype), "GroupQueryAttention must be fp32, fp16 or bf16");
    const bool packed = !n.has_input(1) && !n.has_input(2);
    REQUIRE(packed || (n.has_input(1) && n.has_input(2)), "key and value must both be given");
    REQUIRE(n.has_input(3) == n.has_input(4), "past_key and past_value must both be given");
    // Head size from the query width (attention.rs:1667-1683 for the packed form):
    // the fused kernels take 64 or 128 and the generic ones multiples of 16 up to
    // 256, so anything else is declined here rather than failing at Compute with no
    // CPU fallback.
    REQUIRE(q->dims[2] > 0, "query hidden size must be known");
    const int64_t qheads = packed ? H + 2 * KV : H;
    REQUIRE(q->dims[2] % qheads == 0,
            packed ? "packed QKV hidden size must be divisible by total heads"
                   : "query hidden size must be divisible by num_heads");
    const int64_t qhd = q->dims[2] / qheads;
    REQUIRE(qhd % 16 == 0 && qhd <= 256, "head_size must be a multiple of 16 up to 256");
    if (!packed) {
        auto* k = val(g, n, 1);
        REQUIRE(k && k->has_shape && k->dims.size() == 3 && k->dims[2] == KV * qhd,
                "key hidden size must be kv_num_heads * head_size");
    }
    auto* seq = val(g, n, 5);
    auto* tot = val(g, n, 6);
    REQUIRE(seq && seq->dtype == ONNX_TENSOR_ELEMENT_DATA_TYPE_INT32, "seqlens_k must be int32");
    REQUIRE(tot && tot->dtype == ONNX_TENSOR_ELEMENT_DATA_TYPE_INT32,
            "total_sequence_length must be int32");
    if (n.has_input(3)) {
        auto* pk = val(g, n, 3);
        REQUIRE(pk && pk->has_shape && pk->dims.size() == 4, "past_key must be rank 4");
        REQUIRE(pk->dims[3] == qhd && pk->dims[1] == KV,
                "past_key must be [batch, kv_num_heads, capacity, head_size]");
    }
    // do_rotary defaults to 0 as in ORT's contrib-op schema and CPU kernel (the
    // parity target); the reference defaults it to 1 (attention.rs:1547).
    const bool rotary = n.attr_int("do_rotary", 0) != 0;
    REQUIRE(!rotary || (n.has_input(7) && n.has_input(8)), "do_rotary needs cos/sin caches");
    // Every float input shares the output dtype (attention.rs:1583-1615).
    std::vector<size_t> floats = {0, 1, 2, 3, 4};
    if (rotary) floats.insert(floats.end(), {7, 8});
    floats.insert(floats.end(), {10, 14, 15});
    for (size_t i : floats) {
        if (!n.has_input(i)) continue;
        auto* t = val(g, n, (int)i);
        REQUIRE(t && t->dtype == q->dtype, "GroupQueryAttention float inputs must share one dtype");
    }
    // position_ids only feed the in-op rotary, which is off when do_rotary = 0
    // (attention.rs:1700-1703).
    REQUIRE(!n.has_input(9) || !rotary, "custom position_ids with in-op rotary are not supported");
    if (n.has_input(10)) {  // attention_bias: additive [B or 1, H or 1, S, total] mask
        auto* b = val(g, n, 10);
        REQUIRE(b && b->has_shape && b->dims.size() == 4, "attention_bias must have rank 4");
        REQUIRE(b->dims[1] <= 0 || b->dims[1] == 1 || b->dims[1] == H,
                "attention_bias heads must be 1 or num_heads");
    }
    REQUIRE(!n.has_input(11), "head_sink is not supported");
    REQUIRE(!n.has_input(12) && !n.has_input(13), "quantized KV cache scales are not supported");
    REQUIRE(n.attr_str("k_quant_type", "NONE") == "NONE" &&
                n.attr_str("v_quant_type", "NONE") == "NONE",
            "quantized KV cache is not supported");
    REQUIRE(n.has_input(14) == n.has_input(15),
            "q_norm_weight and k_norm_weight must be provided together");
    for (size_t i : {14, 15})
        if (n.has_input(i)) {
            auto* w = val(g, n, (int)i);
            REQUIRE(w && w->has_shape && w->dims.size() == 1 && w->dims[0] == qhd,
                    "Q/K norm weights must have shape [head_size]");
        }
    // The sliding-window cache (attention.rs:725-880, claim 1552-1575). Otherwise a
    // local_window_size is carried by attention_bias in the reference's Gemma3n
    // form (attention.rs:256-262); without a bias the reference ignores the window
    // while ORT applies it, so that form is declined.
    if (n.attr_int("sliding_window_cache", 0) != 0) {
        const int64_t window = n.attr_int("local_window_size", -1);
        REQUIRE(window > 0, "sliding_window_cache=1 requires local_window_size > 0");
        REQUIRE(!n.has_input(10), "sliding_window_cache is incompatible with attention_bias");
        REQUIRE(n.has_input(3) && n.outputs.size() >= 3 && !n.outputs[1].empty() &&
                    !n.outputs[2].empty(),
                "sliding_window_cache requires past and present key/value");
        auto* pk = val(g, n, 3);
        auto* pv = val(g, n, 4);
        REQUIRE(pk->dims[2] < 0 || pk->dims[2] >= window,
                "sliding-window key cache capacity must be at least local_window_size");
        REQUIRE(!pv || !pv->has_shape || pv->dims.size() != 4 || pv->dims[2] < 0 ||
                    pv->dims[2] >= window,
                "sliding-window value cache capacity must be at least local_window_size");
    } else {
        REQUIRE(n.attr_int("local_window_size", -1) == -1 || n.has_input(10),
                "local_window_size without attention_bias is not supported");
    }
    REQUIRE(n.attr_float("softcap", 0.f) == 0.f, "softcap is not supported");
    REQUIRE(n.attr_int("smooth_softmax", 0) == 0, "smooth_softmax is not supported");
    REQUIRE(n.attr_int("qk_output", 0) == 0, "qk_output is not supported");
    REQUIRE(n.outputs.size() <= 3 || n.outputs[3].empty(), "qk output is not supported");
    return "";
}

// rust/src/ops/attention.rs:2746-2977
std::string claim_paged(const NodeDesc& n, const GraphIR& g) {
    REQUIRE(!n.outputs.empty(), "PagedAttention requires at least 1 output");
    const int64_t H = n.attr_int("num_heads", 0), KV = n.attr_int("kv_num_heads", 0);
    REQUIRE(H > 0 && KV > 0 && H % KV == 0, "bad num_heads/kv_num_heads");
    REQUIRE(n.attr_int("v_head_size", 0) >= 0, "v_head_size must be non-negative");
    REQUIRE(n.attr_int("rotary_offset", 0) >= 0, "rotary_offset must be non-negative");
    REQUIRE(n.attr_float("softcap", 0.f) == 0.f, "softcap is not supported");
    REQUIRE(n.attr_int("local_window_size", -1) == -1, "sliding window is not supported");
    auto* q = val(g, n, 0);
    auto* kc = val(g, n, 3);
    REQUIRE(q && is_float(q->dtype), "PagedAttention must be fp32, fp16 or bf16");
    REQUIRE(kc && kc->has_shape && kc->dims.size() == 4, "key_cache must be [blocks, block, kv, hd]");
    const int64_t hd = kc->dims[3];
    REQUIRE(hd > 0 && hd % 16 == 0 && hd <= 256, "head_size must be a multiple of 16 up to 256");
    for (int i : {5, 6, 7}) {
        auto* t = val(g, n, i);
        REQUIRE(t && t->dtype == ONNX_TENSOR_ELEMENT_DATA_TYPE_INT32,
                "cumulative_sequence_length / past_seqlens / block_table must be int32");
    }
    const bool latent = n.attr_str("kv_cache_layout", "SEPARATE") == "LATENT";
    REQUIRE(latent || (n.has_input(2) && n.has_input(4)), "value and value_cache are required");
    const int64_t vhd = n.attr_int("v_head_size", 0) ? n.attr_int("v_head_size", 0) : hd;
    REQUIRE(vhd == hd || (latent && vhd % 16 == 0 && vhd <= hd),
            "unsupported v_head_size");
    // Query, key and key cache (and value and value cache unless LATENT) share the
    // output's float dtype (attention.rs:2800-2815).
    auto* o = out_val(g, n, 0);
    REQUIRE(!o || o->dtype == q->dtype, "the output must share the query dtype");
    for (int i : {1, 3}) {
        auto* t = val(g, n, i);
        REQUIRE(t && t->dtype == q->dtype, "key and key_cache must share the query dtype");
    }
    if (!latent)
        for (int i : {2, 4}) {
            auto* t = val(g, n, i);
            REQUIRE(t && t->dtype == q->dtype, "value and value_cache must share the query dtype");
        }
    // A cache dtype attribute names the caches' storage; the caches themselves must be
    // the activation dtype (checked above), so only sub-byte packings are declined
    // outright, as the reference does (attention.rs:2759-2765).
    for (const char* k : {"k_cache_dtype", "v_cache_dtype"}) {
        const std::string cd = n.attr_str(k, "");
        REQUIRE(cd != "int4" && cd != "float4e2m1", std::string(k) + " sub-byte packing is unsupported");
    }
    if (n.has_input(10)) {
        auto* sm = val(g, n, 10);
        REQUIRE(sm && sm->dtype == ONNX_TENSOR_ELEMENT_DATA_TYPE_INT32, "slot_mapping must be int32");
    }
    REQUIRE(n.has_input(12) == n.has_input(13), "q/k norm weights must both be given");
    if (n.attr_int("do_rotary", 0) != 0) {
        // attention.rs:2898-2918
        auto *c = val(g, n, 8), *s = val(g, n, 9);
        REQUIRE(c && s && c->dtype == q->dtype && s->dtype == q->dtype,
                "do_rotary=1 requires cos_cache and sin_cache in the output dtype");
        REQUIRE(c->has_shape && c->dims.size() == 2 && c->dims[1] > 0,
                "cos_cache must be [max_position, rotary_dim / 2]");
        const int64_t off = n.attr_int("rotary_offset", 0);
        REQUIRE(off + 2 * c->dims[1] <= hd, "rotary_offset + rotary_dim must not exceed head_size");
    }
    return "";
}

// rust/src/ops/attention.rs:2158-2264. The rotated width is the cos/sin cache's last
// dim (half), as the reference's rope_apply takes it; dims past 2 * half keep their
// values (partial rotary).
std::string claim_rotary(const NodeDesc& n, const GraphIR& g) {
    REQUIRE(!n.outputs.empty() && !n.outputs[0].empty(), "requires an output");
    const bool ms = n.domain == "com.microsoft";
    const int ci = ms ? 2 : 1, si = ms ? 3 : 2, pi = ms ? 1 : 3;
    REQUIRE(n.inputs.size() >= (size_t)(ms ? 4 : 3), "too few inputs");
    auto* x = val(g, n, 0);
    REQUIRE(x && x->has_shape && (x->dims.size() == 3 || x->dims.size() == 4),
            "input must be rank 3 or 4");
    REQUIRE(is_float(x->dtype), "float input required");
    auto *c = val(g, n, ci), *s = val(g, n, si);
    REQUIRE(c && s && c->dtype == x->dtype && s->dtype == x->dtype && c->has_shape &&
                !c->dims.empty(),
            "cos/sin caches must share the input dtype");
    auto* o = g.values.count(n.outputs[0]) ? &g.values.at(n.outputs[0]) : nullptr;
    REQUIRE(!o || o->dtype == 0 || o->dtype == x->dtype, "output must share the input dtype");
    REQUIRE(n.attr_int("is_packed_batching", 0) == 0, "packed batching is not supported");
    const int64_t half = c->dims.back();
    REQUIRE(half > 0, "empty cos cache");
    if (x->dims.size() == 3) {
        const int64_t nh = n.attr_int("num_heads", 0), hidden = x->dims[2];
        if (nh > 0) {
            REQUIRE(hidden > 0 && hidden % nh == 0, "hidden must divide by num_heads");
            REQUIRE(2 * half <= hidden / nh, "rotary width exceeds the head size");
        } else {
            REQUIRE(n.attr_int("rotary_embedding_dim", 0) == 0,
                    "num_heads = 0 needs rotary_embedding_dim = 0 to infer the head size");
            REQUIRE(hidden > 0 && hidden % (2 * half) == 0,
                    "hidden must divide by the inferred head size (2 x cos width)");
        }
    } else if (x->dims[3] > 0) {
        REQUIRE(2 * half <= x->dims[3], "rotary width exceeds the head size");
    }
    const bool has_pos = n.has_input(pi);
    REQUIRE(!ms || has_pos, "com.microsoft RotaryEmbedding requires position_ids");
    if (has_pos) {
        auto* p = val(g, n, pi);
        // The ONNX schemas (ai.onnx opset 23, com.microsoft) type position_ids int64.
        REQUIRE(p && p->dtype == ONNX_TENSOR_ELEMENT_DATA_TYPE_INT64, "position_ids must be int64");
        REQUIRE(p->has_shape && (p->dims.size() == 2 || (ms && p->dims.size() == 1 && p->dims[0] == 1)),
                "position_ids must be [B,S] or, for com.microsoft, [1]");
        REQUIRE(c->dims.size() == 2, "a gathered cos cache must have rank 2");
    } else {
        REQUIRE(c->dims.size() == 3, "without position_ids the cos cache must be [B,S,half]");
    }
    return "";
}

// rust/src/ops/norm.rs:461-523, 571-612
std::string claim_rms(const NodeDesc& n, const GraphIR& g) {
    auto* x = val(g, n, 0);
    REQUIRE(x && is_float(x->dtype), "float input required");
    REQUIRE(n.attr_int("axis", -1) == -1 || (x->has_shape && n.attr_int("axis", -1) ==
                                                                   (int64_t)x->dims.size() - 1),
            "only last-axis normalization is supported");
    if (x->has_shape && !x->dims.empty()) {
        const int64_t D = x->dims.back();
        REQUIRE(D > 0 && D <= 16384, "normalized axis length must be in (0, 16384]");
    }
    if (n.op == "SkipSimplifiedLayerNormalization") {
        auto* sk = val(g, n, 1);
        REQUIRE(sk && sk->dtype == x->dtype, "skip must share the input dtype");
        // mean (output 1) and inv_std_var (output 2) are not produced. Declared but
        // unused, as transformers.js / Mobius exports leave them, the node is claimed
        // (rust/src/ops/norm.rs:586-594); read by any node or a graph output, it is
        // declined, so ORT's own kernel produces them.
        for (size_t i = 1; i <= 2 && i < n.outputs.size(); ++i) {
            const std::string& o = n.outputs[i];
            if (o.empty()) continue;
            bool read = std::find(g.outputs.begin(), g.outputs.end(), o) != g.outputs.end();
            for (const NodeDesc& m : g.nodes)
                for (const std::string& in : m.inputs) read = read || in == o;
            REQUIRE(!read, i == 1 ? "mean output is read" : "inv_std_var output is read");
        }
    } else {
        REQUIRE(n.outputs.size() < 2 || n.outputs[1].empty(), "inv_std_var output is not produced");
    }
    return "";
}

// Decoder glue (rust/src/ops/elementwise.rs:928-980, shape.rs:2453).
std::string claim_binary(const NodeDesc& n, const GraphIR& g) {
    auto *a = val(g, n, 0), *b = val(g, n, 1);
    REQUIRE(a && b && is_float(a->dtype) && a->dtype == b->dtype, "float inputs of one dtype");
    REQUIRE(a->has_shape && b->has_shape && a->dims.size() == b->dims.size(),
            "same-shape operands only (no broadcasting)");
    // Symbolic dims are accepted here; the executor checks the runtime shapes match.
    for (size_t i = 0; i < a->dims.size(); ++i)
        REQUIRE(a->dims[i] < 0 || b->dims[i] < 0 || a->dims[i] == b->dims[i],
                "same-shape operands only (no broadcasting)");
    return "";
}
std::string claim_unary(const NodeDesc& n, const GraphIR& g) {
    auto* a = val(g, n, 0);
    REQUIRE(a && is_float(a->dtype), "float input required");
    return "";
}
std::string claim_cast(const NodeDesc& n, const GraphIR& g) {
    auto* a = val(g, n, 0);
    const int64_t to = n.attr_int("to", 0);
    REQUIRE(a && is_float(a->dtype) && is_float((int)to), "float <-> float casts only");
    return "";
}
std::string claim_gather(const NodeDesc& n, const GraphIR& g) {
    auto *d = val(g, n, 0), *i = val(g, n, 1);
    REQUIRE(n.attr_int("axis", 0) == 0, "axis 0 only");
    REQUIRE(d && d->has_shape && d->dims.size() == 2 && is_float(d->dtype), "2-D float table only");
    REQUIRE(i && i->dtype == ONNX_TENSOR_ELEMENT_DATA_TYPE_INT64, "int64 indices only");
    return "";
}

// rust/src/ops/reduction.rs:582-630 (registered at :962). The reference claims any
// numeric dtype, axis and select_last_index; the kernel here reduces contiguous
// float rows with the lowest index winning ties, so other forms are declined.
std::string claim_argmax(const NodeDesc& n, const GraphIR& g) {
    REQUIRE(n.inputs.size() == 1 && n.outputs.size() == 1 && !n.outputs[0].empty(),
            "requires 1 input and 1 output");
    auto* x = val(g, n, 0);
    REQUIRE(x && is_float(x->dtype), "float input required");
    REQUIRE(x->has_shape && !x->dims.empty(), "input rank must be known and at least 1");
    const int64_t r = (int64_t)x->dims.size();
    int64_t axis = n.attr_int("axis", 0);
    if (axis < 0) axis += r;
    REQUIRE(axis >= 0 && axis < r, "axis out of range");
    const int64_t kd = n.attr_int("keepdims", 1);
    REQUIRE(kd == 0 || kd == 1, "keepdims must be 0 or 1");
    const int64_t last = n.attr_int("select_last_index", 0);
    REQUIRE(last == 0 || last == 1, "select_last_index must be 0 or 1");
    REQUIRE(x->dims[axis] != 0, "the reduced axis is empty");
    auto* out = out_val(g, n, 0);
    REQUIRE(!out || out->dtype == ONNX_TENSOR_ELEMENT_DATA_TYPE_INT64, "output must be int64");
    return "";
}

// rust/src/ops/quant.rs:1713-1749
std::string claim_gbq(const NodeDesc& n, const GraphIR& g) {
    REQUIRE(!n.outputs.empty() && !n.outputs[0].empty(), "requires at least one output");
    auto* out = out_val(g, n, 0);
    REQUIRE(out, "missing output type/shape info");
    auto *d = val(g, n, 0), *i = val(g, n, 1), *s = val(g, n, 2);
    REQUIRE(d && i && s, "missing tensor type/shape info on an input");
    REQUIRE(d->dtype == ONNX_TENSOR_ELEMENT_DATA_TYPE_UINT8 &&
                (i->dtype == ONNX_TENSOR_ELEMENT_DATA_TYPE_INT32 ||
                 i->dtype == ONNX_TENSOR_ELEMENT_DATA_TYPE_INT64) &&
                s->dtype == out->dtype && is_float(s->dtype),
            "data must be uint8, indices int32/int64, and scales/output the same float dtype");
    if (n.has_input(3)) {
        auto* zp = val(g, n, 3);
        REQUIRE(zp && zp->dtype == ONNX_TENSOR_ELEMENT_DATA_TYPE_UINT8,
                "zero_points must be uint8 when present");
    }
    REQUIRE(n.attr_int("bits", 4) == 4, "only 4-bit data is supported");
    REQUIRE(n.attr_int("gather_axis", 0) == 0 && n.attr_int("quantize_axis", 1) == 1,
            "only gather_axis=0 and quantize_axis=1 are supported");
    REQUIRE(n.attr_int("block_size", 128) >= 16, "block_size must be at least 16");
    // The kernel's table layout (the reference reads data as [V, D/2] too).
    REQUIRE(!d->has_shape || d->dims.size() == 2, "data must be rank 2");
    return "";
}

struct Entry {
    const char* domain;
    const char* op;
    ClaimFn fn;
};
const Entry kRegistry[] = {
    {"com.microsoft", "MatMulNBits", claim_matmulnbits},
    {"com.microsoft", "GatherBlockQuantized", claim_gbq},
    {"com.microsoft", "GroupQueryAttention", claim_gqa},
    {"com.microsoft", "PagedAttention", claim_paged},
    {"com.microsoft", "RotaryEmbedding", claim_rotary},
    {"", "RotaryEmbedding", claim_rotary},
    {"com.microsoft", "SimplifiedLayerNormalization", claim_rms},
    {"com.microsoft", "SkipSimplifiedLayerNormalization", claim_rms},
    // Some exporters stamp SimplifiedLayerNormalization into the default domain
    // (rust/src/ops/norm.rs:930-968).
    {"", "SimplifiedLayerNormalization", claim_rms},
    {"", "RMSNormalization", claim_rms},
    {"", "Add", claim_binary},
    {"", "Mul", claim_binary},
    {"", "Sub", claim_binary},
    {"", "Sigmoid", claim_unary},
    {"", "Cast", claim_cast},
    {"", "Gather", claim_gather},
    {"", "ArgMax", claim_argmax},
};

}  // namespace

ClaimFn find_claim(const std::string& domain, const std::string& op) {
    for (const auto& e : kRegistry)
        if (domain == e.domain && op == e.op) return e.fn;
    return nullptr;
}

std::string claim_reason(const NodeDesc& n, const GraphIR& g) {
    ClaimFn fn = find_claim(n.domain, n.op);
    if (!fn) return "no MI355X kernel for " + (n.domain.empty() ? "" : n.domain + ".") + n.op;
    return fn(n, g);
}

// --------------------------------------------------------------- clusters --

namespace {
struct Bits {
    std::vector<uint64_t> w;
    explicit Bits(size_t n = 0) : w((n + 63) / 64, 0) {}
    void set(size_t i) { w[i >> 6] |= 1ull << (i & 63); }
    bool get(size_t i) const { return (w[i >> 6] >> (i & 63)) & 1; }
    void operator|=(const Bits& o) {
        for (size_t i = 0; i < w.size(); ++i) w[i] |= o.w[i];
    }
    bool intersects(const Bits& o) const {
        for (size_t i = 0; i < w.size(); ++i)
            if (w[i] & o.w[i]) return true;
        return false;
    }
};
}  // namespace

std::vector<std::vector<size_t>> build_clusters(const GraphIR& g,
                                                const std::vector<bool>& claimed) {
    const size_t N = g.nodes.size();
    // Producer of each value; data edges producer -> consumer.
    std::map<std::string, size_t> producer;
    for (size_t i = 0; i < N; ++i)
        for (const auto& o : g.nodes[i].outputs)
            if (!o.empty()) producer[o] = i;
    std::vector<std::vector<size_t>> preds(N), succs(N);
    for (size_t i = 0; i < N; ++i)
        for (const auto& in : g.nodes[i].inputs) {
            auto it = in.empty() ? producer.end() : producer.find(in);
            if (it != producer.end() && it->second != i) {
                preds[i].push_back(it->second);
                succs[it->second].push_back(i);
            }
        }
    // Topological order (ORT hands nodes in topological order; recompute to be safe).
    std::vector<int> indeg(N, 0);
    for (size_t i = 0; i < N; ++i) indeg[i] = (int)preds[i].size();
    std::vector<size_t> order, ready;
    for (size_t i = 0; i < N; ++i)
        if (!indeg[i]) ready.push_back(i);
    while (!ready.empty()) {
        std::sort(ready.begin(), ready.end(), std::greater<size_t>());
        size_t v = ready.back();
        ready.pop_back();
        order.push_back(v);
        for (size_t s : succs[v])
            if (--indeg[s] == 0) ready.push_back(s);
    }
    if (order.size() != N) fail("graph has a cycle", ORT_INVALID_GRAPH);
    // Ancestor / descendant reachability bitsets (rust/src/ep.rs:749-756).
    std::vector<Bits> anc(N, Bits(N)), desc(N, Bits(N));
    for (size_t v : order)
        for (size_t p : preds[v]) {
            anc[v].set(p);
            anc[v] |= anc[p];
        }
    for (auto it = order.rbegin(); it != order.rend(); ++it)
        for (size_t s : succs[*it]) {
            desc[*it].set(s);
            desc[*it] |= desc[s];
        }
    std::vector<int> cluster(N, -1);
    std::vector<Bits> members;
    // A set is convex when no outside node is both reachable from it and reaches
    // it (rust/src/ep.rs:782-795).
    auto convex = [&](const Bits& m) {
        for (size_t u = 0; u < N; ++u)
            if (!m.get(u) && anc[u].intersects(m) && desc[u].intersects(m)) return false;
        return true;
    };
    // The quotient graph (clusters contracted, other nodes alone) must stay
    // acyclic (rust/src/ep.rs:842-891).
    auto quotient_acyclic = [&](const std::vector<int>& cl) {
        const size_t C = members.size();
        auto qid = [&](size_t v) { return cl[v] >= 0 ? (size_t)cl[v] : C + v; };
        std::vector<std::vector<size_t>> qs(C + N);
        std::vector<int> qin(C + N, 0);
        std::vector<bool> used(C + N, false);
        for (size_t v = 0; v < N; ++v) {
            used[qid(v)] = true;
            for (size_t s : succs[v]) {
                size_t a = qid(v), b = qid(s);
                if (a != b) {
                    qs[a].push_back(b);
                    qin[b]++;
                }
            }
        }
        std::vector<size_t> st;
        size_t seen = 0, total = 0;
        for (size_t q = 0; q < C + N; ++q)
            if (used[q]) {
                ++total;
                if (!qin[q]) st.push_back(q);
            }
        while (!st.empty()) {
            size_t q = st.back();
            st.pop_back();
            ++seen;
            for (size_t b : qs[q])
                if (--qin[b] == 0) st.push_back(b);
        }
        return seen == total;
    };
    // Start from singletons and merge along data edges between claimed nodes until
    // nothing changes (rust/src/ep.rs:760-822). Unlike a merge-then-repair pass,
    // a merge is only taken when the merged set is convex AND the contracted
    // graph stays acyclic, so no cluster ever has to be dropped back to the CPU.
    for (size_t v = 0; v < N; ++v)
        if (claimed[v]) {
            cluster[v] = (int)members.size();
            Bits m(N);
            m.set(v);
            members.push_back(m);
        }
    std::vector<std::pair<size_t, size_t>> edges;
    for (size_t u : order)
        if (claimed[u])
            for (size_t v : succs[u])
                if (claimed[v]) edges.emplace_back(u, v);
    for (bool changed = true; changed;) {
        changed = false;
        for (auto [u, v] : edges) {
            const int cu = cluster[u], cv = cluster[v];
            if (cu == cv) continue;
            Bits m = members[cu];
            m |= members[cv];
            if (!convex(m)) continue;
            std::vector<int> trial = cluster;
            for (size_t x = 0; x < N; ++x)
                if (trial[x] == cv) trial[x] = cu;
            if (!quotient_acyclic(trial)) continue;
            cluster = std::move(trial);
            members[cu] = m;
            members[cv] = Bits(N);
            changed = true;
        }
    }
    std::vector<std::vector<size_t>> out(members.size());
    for (size_t v : order)
        if (cluster[v] >= 0) out[cluster[v]].push_back(v);
    out.erase(std::remove_if(out.begin(), out.end(), [](auto& c) { return c.empty(); }), out.end());
    // Clusters in topological order of their first node.
    std::vector<size_t> pos(N);
    for (size_t i = 0; i < N; ++i) pos[order[i]] = i;
    std::sort(out.begin(), out.end(),
              [&](const auto& a, const auto& b) { return pos[a[0]] < pos[b[0]]; });
    return out;
}

// ------------------------------------------- layer groups of large decoders --

namespace {
void put_utf8(uint32_t cp, std::string* out) {
    if (cp < 0x80) {
        out->push_back((char)cp);
    } else if (cp < 0x800) {
        out->push_back((char)(0xC0 | (cp >> 6)));
        out->push_back((char)(0x80 | (cp & 0x3F)));
    } else if (cp < 0x10000) {
        out->push_back((char)(0xE0 | (cp >> 12)));
        out->push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
        out->push_back((char)(0x80 | (cp & 0x3F)));
    } else {
        out->push_back((char)(0xF0 | (cp >> 18)));
        out->push_back((char)(0x80 | ((cp >> 12) & 0x3F)));
        out->push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
        out->push_back((char)(0x80 | (cp & 0x3F)));
    }
}

// Recursive-descent reader over the JSON grammar's array-of-strings subset.
struct JsonStrings {
    const std::string& t;
    size_t i = 0;
    void ws() {
        while (i < t.size() && (t[i] == ' ' || t[i] == '\t' || t[i] == '\n' || t[i] == '\r')) ++i;
    }
    bool hex4(uint32_t* v) {
        if (i + 4 > t.size()) return false;
        *v = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = t[i++];
            *v <<= 4;
            if (c >= '0' && c <= '9') *v |= (uint32_t)(c - '0');
            else if (c >= 'a' && c <= 'f') *v |= (uint32_t)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') *v |= (uint32_t)(c - 'A' + 10);
            else return false;
        }
        return true;
    }
    bool str(std::string* out) {
        if (i >= t.size() || t[i] != '"') return false;
        ++i;
        while (i < t.size()) {
            const unsigned char c = (unsigned char)t[i++];
            if (c == '"') return true;
            if (c < 0x20) return false;  // control characters must be escaped
            if (c != '\\') {
                out->push_back((char)c);
                continue;
            }
            if (i >= t.size()) return false;
            const char e = t[i++];
            switch (e) {
                case '"': out->push_back('"'); break;
                case '\\': out->push_back('\\'); break;
                case '/': out->push_back('/'); break;
                case 'b': out->push_back('\b'); break;
                case 'f': out->push_back('\f'); break;
                case 'n': out->push_back('\n'); break;
                case 'r': out->push_back('\r'); break;
                case 't': out->push_back('\t'); break;
                case 'u': {
                    uint32_t cp;
                    if (!hex4(&cp)) return false;
                    if (cp >= 0xD800 && cp < 0xDC00) {  // high surrogate: a low one follows
                        uint32_t lo;
                        if (i + 2 > t.size() || t[i] != '\\' || t[i + 1] != 'u') return false;
                        i += 2;
                        if (!hex4(&lo) || lo < 0xDC00 || lo >= 0xE000) return false;
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    } else if (cp >= 0xDC00 && cp < 0xE000) {
                        return false;
                    }
                    put_utf8(cp, out);
                    break;
                }
                default: return false;
            }
        }
        return false;  // unterminated
    }
};
}  // namespace

bool parse_json_string_array(const std::string& text, std::vector<std::string>* out) {
    JsonStrings p{text};
    std::vector<std::string> items;
    p.ws();
    if (p.i >= text.size() || text[p.i] != '[') return false;
    ++p.i;
    p.ws();
    if (p.i < text.size() && text[p.i] == ']') {
        ++p.i;
    } else {
        for (;;) {
            p.ws();
            std::string s;
            if (!p.str(&s)) return false;
            items.push_back(std::move(s));
            p.ws();
            if (p.i >= text.size()) return false;
            if (text[p.i] == ',') {
                ++p.i;
                continue;
            }
            if (text[p.i] != ']') return false;
            ++p.i;
            break;
        }
    }
    p.ws();
    if (p.i != text.size()) return false;
    *out = std::move(items);
    return true;
}

namespace {
bool is_attention_anchor(const NodeDesc& n) {
    if (n.domain == "com.microsoft" && n.op == "PagedAttention") return true;
    const bool presents = n.outputs.size() >= 3 && !n.outputs[1].empty() && !n.outputs[2].empty();
    if (!presents) return false;
    if (n.domain == "com.microsoft") return n.op == "GroupQueryAttention" || n.op == "MultiHeadAttention";
    return (n.domain.empty() || n.domain == "ai.onnx") && n.op == "Attention";
}
}  // namespace

std::set<std::string> infer_layer_boundaries(const GraphIR& g) {
    const size_t N = g.nodes.size();
    std::map<std::string, size_t> producer;
    std::vector<size_t> anchors;
    for (size_t i = 0; i < N; ++i) {
        if (is_attention_anchor(g.nodes[i])) anchors.push_back(i);
        for (const auto& o : g.nodes[i].outputs)
            if (!o.empty()) producer.emplace(o, i);  // first producer wins
    }
    if (anchors.size() < 2) return {};
    std::vector<std::vector<size_t>> succs(N), preds(N);
    for (size_t i = 0; i < N; ++i) {
        std::set<size_t> seen;
        for (const auto& in : g.nodes[i].inputs) {
            auto it = in.empty() ? producer.end() : producer.find(in);
            if (it == producer.end() || it->second == i || !seen.insert(it->second).second) continue;
            succs[it->second].push_back(i);
            preds[i].push_back(it->second);
        }
    }
    std::set<std::string> out;
    std::vector<char> down(N), up(N);
    for (size_t a = 0; a + 1 < anchors.size(); ++a) {
        const size_t cur = anchors[a], next = anchors[a + 1];
        // Nodes in graph order up to `next` reached from `cur`, and nodes from `cur`
        // on that reach `next`.
        std::fill(down.begin(), down.end(), 0);
        std::fill(up.begin(), up.end(), 0);
        std::vector<size_t> stack{cur};
        while (!stack.empty()) {
            const size_t v = stack.back();
            stack.pop_back();
            for (size_t s : succs[v])
                if (s <= next && !down[s]) {
                    down[s] = 1;
                    stack.push_back(s);
                }
        }
        stack.assign(1, next);
        while (!stack.empty()) {
            const size_t v = stack.back();
            stack.pop_back();
            for (size_t p : preds[v])
                if (p >= cur && !up[p]) {
                    up[p] = 1;
                    stack.push_back(p);
                }
        }
        size_t hit = 0;
        for (size_t k = next; k-- > cur + 1;)
            if (g.nodes[k].op == "Add" && down[k] && up[k]) {
                hit = k;
                break;
            }
        if (!hit) return {};  // one layer without a residual Add: no boundaries at all
        if (!g.nodes[hit].outputs.empty() && !g.nodes[hit].outputs[0].empty())
            out.insert(g.nodes[hit].outputs[0]);
    }
    return out;
}

size_t select_layer_span(const char* value) {
    if (!value) return 0;  // auto: whole at any depth
    std::string v(value);
    const auto b = v.find_first_not_of(" \t\n\r");
    if (b == std::string::npos) return 0;
    v = v.substr(b, v.find_last_not_of(" \t\n\r") - b + 1);
    if (v == "auto" || v == "0" || v == "off" || v == "false") return 0;
    size_t i = v[0] == '+' ? 1 : 0;
    if (i == v.size() || v.size() - i > 18) return 0;
    size_t span = 0;
    for (; i < v.size(); ++i) {
        if (v[i] < '0' || v[i] > '9') return 0;
        span = span * 10 + (size_t)(v[i] - '0');
    }
    return span;
}

std::vector<std::vector<size_t>> split_layer_clusters(const GraphIR& g,
                                                      std::vector<std::vector<size_t>> clusters,
                                                      const std::set<std::string>& boundaries,
                                                      size_t span) {
    if (!span || boundaries.empty()) return clusters;
    std::vector<std::vector<size_t>> out;
    for (auto& cl : clusters) {
        std::vector<size_t> part;
        size_t layers = 0;
        for (size_t v : cl) {
            part.push_back(v);
            bool ends = false;
            for (const auto& o : g.nodes[v].outputs) ends = ends || (!o.empty() && boundaries.count(o));
            if (ends && ++layers == span) {
                out.push_back(std::move(part));
                part.clear();
                layers = 0;
            }
        }
        if (!part.empty()) out.push_back(std::move(part));
    }
    return out;
}

}  // namespace ortmi_ep
