// In-process harness host for plugin execution providers.
//
// ONNX Runtime itself is not available to this project, so this file plays its
// part on the plugin ABI: it implements the OrtApi / OrtEpApi slots listed in
// include/ort_plugin_ep_abi.h over an in-memory graph, loads an EP library with
// dlopen, and drives CreateEpFactories -> GetSupportedDevices -> CreateEp ->
// GetCapability -> Compile -> CreateState/Compute the way ORT's plugin loader
// does (the reference's call sequence: rust/src/lib.rs:90-155,
// rust/src/factory.rs:116-213, rust/src/ep.rs:119-357, 928-1211, 1931-2134).
// Graphs must be claimed completely: there is no CPU execution provider here.
// Placement follows ORT's rule for a fused node: its inputs and outputs live on
// the EP's default memory device (OrtEp::GetDefaultMemoryDevice; null = CPU
// memory). A feed on the other side (host vs device) is copied there through the
// EP factory's data transfer before Compute, into a buffer from the allocator the
// factory hands out for the memory info the EP device registered; an output bound
// to memory on the other side is produced in such a buffer and copied back after
// Compute; an output nobody binds is allocated on the EP's side. A feed or binding
// already on the EP's side (device buffers with an HBM EP: the IOBinding case) is
// used in place.
#include <dlfcn.h>
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <set>
#include <string>
#include <type_traits>
#include <unordered_map>
#include <vector>

#include "../../../include/ort_plugin_ep_abi.h"

// ----------------------------------------------------------- host objects --
struct OrtStatus {
    OrtErrorCode code;
    std::string msg;
};
struct OrtHardwareDevice {
    OrtHardwareDeviceType type;
};
struct OrtEpDevice {
    OrtEpFactory* factory;
    const OrtHardwareDevice* device;
    std::vector<const OrtMemoryInfo*> allocator_infos;  // EpDevice_AddAllocatorInfo (not owned)
};
// Where memory lives (ORT's OrtDevice): type, vendor id, device id, memory type.
struct OrtMemoryDevice {
    OrtMemoryInfoDeviceType type = OrtMemoryInfoDeviceType_CPU;
    uint32_t vendor = 0;
    int32_t id = 0;
    OrtDeviceMemoryType mem = OrtDeviceMemoryType_DEFAULT;
};
// Type/shape info; the same object serves as OrtTypeInfo and as the tensor info.
struct OrtTensorTypeAndShapeInfo {
    int dtype = 0;
    std::vector<int64_t> dims;
};
struct OrtTypeInfo : OrtTensorTypeAndShapeInfo {};
struct OrtValue {
    OrtTensorTypeAndShapeInfo info;
    void* data = nullptr;       // device pointer (or host for initializers)
    std::vector<uint8_t> host;  // initializer storage
    bool on_device = false;     // where `data` lives (GPU memory or host memory)
};
struct OrtValueInfo {
    std::string name;
    OrtTypeInfo type;
    bool is_initializer = false;
    OrtValue init;  // initializer value (host memory)
    const OrtNode* producer = nullptr;
    size_t producer_output = 0;
};
struct OrtOpAttr {
    std::string name;
    OrtOpAttrType type = ORT_OP_ATTR_UNDEFINED;
    int64_t i = 0;
    float f = 0.f;
    std::string s;
    std::vector<int64_t> ints;
    std::vector<float> floats;
};
struct OrtNode {
    size_t id = 0;
    std::string name, op, domain;
    int since = 1;
    std::vector<OrtValueInfo*> inputs, outputs;
    std::vector<std::unique_ptr<OrtOpAttr>> attrs;
};
struct OrtGraph {
    std::vector<OrtNode*> nodes;
    std::vector<OrtValueInfo*> inputs, outputs, initializers;
    std::map<std::string, std::string> metadata;  // the model's custom metadata map
    const OrtNode* parent = nullptr;              // set for a control-flow body
};
struct OrtModelMetadata {
    std::map<std::string, std::string> custom;
};
struct OrtEpGraphSupportInfo {
    std::vector<std::vector<const OrtNode*>> groups;
};
struct OrtKernelContext {
    std::vector<OrtValue*> inputs;
    std::vector<const OrtValueInfo*> outputs;  // the fused node's outputs (name, type)
    struct Session* session;
};
struct OrtNodeComputeContext {
    std::string name;
};
struct OrtMemoryInfo {
    std::string name;
    OrtAllocatorType type = OrtDeviceAllocator;
    int id = 0;
    OrtMemType mem_type = OrtMemTypeDefault;
    OrtMemoryDevice device;
    size_t alignment = 0;
};

namespace {

thread_local std::string g_err;

OrtStatus* mk(OrtErrorCode c, const std::string& m) { return new OrtStatus{c, m}; }

// ------------------------------------------------------------ OrtApi impl --
OrtStatus* h_CreateStatus(OrtErrorCode code, const char* msg) { return mk(code, msg ? msg : ""); }
OrtErrorCode h_GetErrorCode(const OrtStatus* s) { return s ? s->code : ORT_OK; }
const char* h_GetErrorMessage(const OrtStatus* s) { return s ? s->msg.c_str() : ""; }
void h_ReleaseStatus(OrtStatus* s) { delete s; }
OrtStatus* h_GetTensorMutableData(OrtValue* v, void** out) {
    *out = v->data;
    return nullptr;
}
OrtStatus* h_GetTensorData(const OrtValue* v, const void** out) {
    *out = v->data;
    return nullptr;
}
OrtStatus* h_CastTypeInfoToTensorInfo(const OrtTypeInfo* t, const OrtTensorTypeAndShapeInfo** out) {
    *out = t;
    return nullptr;
}
OrtStatus* h_GetOnnxTypeFromTypeInfo(const OrtTypeInfo*, ONNXType* out) {
    *out = ONNX_TYPE_TENSOR;
    return nullptr;
}
OrtStatus* h_GetTensorElementType(const OrtTensorTypeAndShapeInfo* t, ONNXTensorElementDataType* out) {
    *out = (ONNXTensorElementDataType)t->dtype;
    return nullptr;
}
OrtStatus* h_GetDimensionsCount(const OrtTensorTypeAndShapeInfo* t, size_t* out) {
    *out = t->dims.size();
    return nullptr;
}
OrtStatus* h_GetDimensions(const OrtTensorTypeAndShapeInfo* t, int64_t* dims, size_t len) {
    for (size_t i = 0; i < len && i < t->dims.size(); ++i) dims[i] = t->dims[i];
    return nullptr;
}
OrtStatus* h_GetTensorShapeElementCount(const OrtTensorTypeAndShapeInfo* t, size_t* out) {
    size_t n = 1;
    for (auto d : t->dims) n *= (size_t)(d < 0 ? 0 : d);
    *out = n;
    return nullptr;
}
OrtStatus* h_GetTensorTypeAndShape(const OrtValue* v, OrtTensorTypeAndShapeInfo** out) {
    *out = new OrtTensorTypeAndShapeInfo(v->info);
    return nullptr;
}
void h_ReleaseTensorTypeAndShapeInfo(OrtTensorTypeAndShapeInfo* t) { delete t; }
OrtStatus* h_CreateMemoryInfo(const char* name, OrtAllocatorType type, int id, OrtMemType mem_type,
                              OrtMemoryInfo** out) {
    if (!name || !out) return mk(ORT_INVALID_ARGUMENT, "CreateMemoryInfo: null argument");
    auto* m = new OrtMemoryInfo();
    m->name = name;
    m->type = type;
    m->id = id;
    m->mem_type = mem_type;
    // ORT's names: "Cpu" is host memory; this harness reads any other as GPU memory.
    if (std::strcmp(name, "Cpu") != 0) m->device = {OrtMemoryInfoDeviceType_GPU, 0x1002, id, {}};
    *out = m;
    return nullptr;
}
OrtStatus* h_CreateMemoryInfo_V2(const char* name, OrtMemoryInfoDeviceType device_type,
                                 uint32_t vendor_id, int32_t device_id, OrtDeviceMemoryType mem_type,
                                 size_t alignment, OrtAllocatorType allocator_type,
                                 OrtMemoryInfo** out) {
    if (!name || !out) return mk(ORT_INVALID_ARGUMENT, "CreateMemoryInfo_V2: null argument");
    if (device_type != OrtMemoryInfoDeviceType_CPU && device_type != OrtMemoryInfoDeviceType_GPU)
        return mk(ORT_INVALID_ARGUMENT, "CreateMemoryInfo_V2: device type not supported here");
    auto* m = new OrtMemoryInfo();
    m->name = name;
    m->type = allocator_type;
    m->id = device_id;
    m->device = {device_type, vendor_id, device_id, mem_type};
    m->alignment = alignment;
    *out = m;
    return nullptr;
}
OrtStatus* h_MemoryInfoGetName(const OrtMemoryInfo* m, const char** out) {
    *out = m->name.c_str();
    return nullptr;
}
OrtStatus* h_MemoryInfoGetId(const OrtMemoryInfo* m, int* out) {
    *out = m->id;
    return nullptr;
}
void h_ReleaseMemoryInfo(OrtMemoryInfo* m) { delete m; }
OrtStatus* h_KernelContext_GetInputCount(const OrtKernelContext* c, size_t* out) {
    *out = c->inputs.size();
    return nullptr;
}
OrtStatus* h_KernelContext_GetOutputCount(const OrtKernelContext* c, size_t* out) {
    *out = c->outputs.size();
    return nullptr;
}
OrtStatus* h_KernelContext_GetInput(const OrtKernelContext* c, size_t i, const OrtValue** out) {
    if (i >= c->inputs.size()) return mk(ORT_INVALID_ARGUMENT, "input index out of range");
    *out = c->inputs[i];
    return nullptr;
}
OrtStatus* h_KernelContext_GetOutput(OrtKernelContext* c, size_t i, const int64_t* dims,
                                     size_t n, OrtValue** out);  // defined after Session
const OrtEpApi* h_GetEpApi();
OrtHardwareDeviceType h_HardwareDevice_Type(const OrtHardwareDevice* d) { return d->type; }
OrtStatus* h_GetValueInfoName(const OrtValueInfo* v, const char** name) {
    *name = v->name.c_str();
    return nullptr;
}
OrtStatus* h_GetValueInfoTypeInfo(const OrtValueInfo* v, const OrtTypeInfo** t) {
    *t = &v->type;
    return nullptr;
}
OrtStatus* h_ValueInfo_GetValueProducer(const OrtValueInfo* v, const OrtNode** p, size_t* idx) {
    *p = v->producer;
    if (idx) *idx = v->producer_output;
    return nullptr;
}
OrtStatus* h_ValueInfo_GetInitializerValue(const OrtValueInfo* v, const OrtValue** out) {
    *out = v->is_initializer ? &v->init : nullptr;
    return nullptr;
}
OrtStatus* h_ValueInfo_IsConstantInitializer(const OrtValueInfo* v, bool* out) {
    *out = v->is_initializer;
    return nullptr;
}
#define LIST_FNS(NAME, FIELD, T)                                                      \
    OrtStatus* h_Graph_GetNum##NAME(const OrtGraph* g, size_t* out) {                 \
        *out = g->FIELD.size();                                                       \
        return nullptr;                                                               \
    }                                                                                 \
    OrtStatus* h_Graph_Get##NAME(const OrtGraph* g, const T** out, size_t num) {      \
        for (size_t i = 0; i < num && i < g->FIELD.size(); ++i) out[i] = g->FIELD[i]; \
        return nullptr;                                                               \
    }
LIST_FNS(Inputs, inputs, OrtValueInfo)
LIST_FNS(Outputs, outputs, OrtValueInfo)
LIST_FNS(Initializers, initializers, OrtValueInfo)
LIST_FNS(Nodes, nodes, OrtNode)
#undef LIST_FNS
OrtStatus* h_Graph_GetParentNode(const OrtGraph* g, const OrtNode** node) {
    *node = g->parent;
    return nullptr;
}
OrtStatus* h_Graph_GetModelMetadata(const OrtGraph* g, OrtModelMetadata** out) {
    *out = new OrtModelMetadata{g->metadata};
    return nullptr;
}
OrtStatus* h_ModelMetadataLookupCustomMetadataMap(const OrtModelMetadata* md, OrtAllocator* alloc,
                                                  const char* key, char** value) {
    *value = nullptr;
    auto it = md->custom.find(key);
    if (it == md->custom.end()) return nullptr;
    char* p = static_cast<char*>(alloc->Alloc(alloc, it->second.size() + 1));
    if (!p) return mk(ORT_FAIL, "allocation failed");
    std::memcpy(p, it->second.c_str(), it->second.size() + 1);
    *value = p;
    return nullptr;
}
void h_ReleaseModelMetadata(OrtModelMetadata* md) { delete md; }
void* default_alloc(OrtAllocator*, size_t n) { return std::malloc(n); }
void default_free(OrtAllocator*, void* p) { std::free(p); }
OrtStatus* h_GetAllocatorWithDefaultOptions(OrtAllocator** out) {
    static OrtAllocator cpu = [] {
        OrtAllocator a{};
        a.version = ORT_API_VERSION;
        a.Alloc = default_alloc;
        a.Free = default_free;
        return a;
    }();
    *out = &cpu;
    return nullptr;
}
OrtStatus* h_Node_GetId(const OrtNode* n, size_t* id) {
    *id = n->id;
    return nullptr;
}
OrtStatus* h_Node_GetName(const OrtNode* n, const char** s) {
    *s = n->name.c_str();
    return nullptr;
}
OrtStatus* h_Node_GetOperatorType(const OrtNode* n, const char** s) {
    *s = n->op.c_str();
    return nullptr;
}
OrtStatus* h_Node_GetDomain(const OrtNode* n, const char** s) {
    *s = n->domain.c_str();
    return nullptr;
}
OrtStatus* h_Node_GetSinceVersion(const OrtNode* n, int* v) {
    *v = n->since;
    return nullptr;
}
OrtStatus* h_Node_GetNumInputs(const OrtNode* n, size_t* out) {
    *out = n->inputs.size();
    return nullptr;
}
OrtStatus* h_Node_GetInputs(const OrtNode* n, const OrtValueInfo** out, size_t num) {
    for (size_t i = 0; i < num && i < n->inputs.size(); ++i) out[i] = n->inputs[i];
    return nullptr;
}
OrtStatus* h_Node_GetNumOutputs(const OrtNode* n, size_t* out) {
    *out = n->outputs.size();
    return nullptr;
}
OrtStatus* h_Node_GetOutputs(const OrtNode* n, const OrtValueInfo** out, size_t num) {
    for (size_t i = 0; i < num && i < n->outputs.size(); ++i) out[i] = n->outputs[i];
    return nullptr;
}
OrtStatus* h_Node_GetNumAttributes(const OrtNode* n, size_t* out) {
    *out = n->attrs.size();
    return nullptr;
}
OrtStatus* h_Node_GetAttributes(const OrtNode* n, const OrtOpAttr** out, size_t num) {
    for (size_t i = 0; i < num && i < n->attrs.size(); ++i) out[i] = n->attrs[i].get();
    return nullptr;
}
OrtStatus* h_Node_GetAttributeByName(const OrtNode* n, const char* name, const OrtOpAttr** out) {
    *out = nullptr;
    for (auto& a : n->attrs)
        if (a->name == name) {
            *out = a.get();
            return nullptr;
        }
    return mk(ORT_NOT_FOUND, std::string("attribute not found: ") + name);
}
OrtStatus* h_OpAttr_GetType(const OrtOpAttr* a, OrtOpAttrType* t) {
    *t = a->type;
    return nullptr;
}
OrtStatus* h_OpAttr_GetName(const OrtOpAttr* a, const char** s) {
    *s = a->name.c_str();
    return nullptr;
}
OrtStatus* h_ReadOpAttr(const OrtOpAttr* a, OrtOpAttrType t, void* data, size_t len, size_t* out) {
    if (t != a->type) return mk(ORT_INVALID_ARGUMENT, "attribute type mismatch");
    const void* src = nullptr;
    size_t need = 0;
    switch (t) {
        case ORT_OP_ATTR_INT: src = &a->i; need = 8; break;
        case ORT_OP_ATTR_FLOAT: src = &a->f; need = 4; break;
        case ORT_OP_ATTR_STRING: src = a->s.data(); need = a->s.size(); break;
        case ORT_OP_ATTR_INTS: src = a->ints.data(); need = a->ints.size() * 8; break;
        case ORT_OP_ATTR_FLOATS: src = a->floats.data(); need = a->floats.size() * 4; break;
        default: return mk(ORT_NOT_IMPLEMENTED, "attribute type");
    }
    *out = need;
    if (len < need) return mk(ORT_INVALID_ARGUMENT, "buffer too small");
    if (need) std::memcpy(data, src, need);
    return nullptr;
}

// ---------------------------------------------------------- OrtEpApi impl --
OrtStatus* h_CreateEpDevice(OrtEpFactory* f, const OrtHardwareDevice* d, const OrtKeyValuePairs*,
                            const OrtKeyValuePairs*, OrtEpDevice** out) {
    *out = new OrtEpDevice{f, d, {}};
    return nullptr;
}
void h_ReleaseEpDevice(OrtEpDevice* d) { delete d; }
OrtStatus* h_EpGraphSupportInfo_AddNodesToFuse(OrtEpGraphSupportInfo* info,
                                               const OrtNode* const* nodes, size_t n,
                                               const OrtNodeFusionOptions* opts) {
    if (!opts || opts->ort_version_supported < 1) return mk(ORT_INVALID_ARGUMENT, "bad fusion options");
    info->groups.emplace_back(nodes, nodes + n);
    return nullptr;
}
OrtStatus* h_EpGraphSupportInfo_AddSingleNode(OrtEpGraphSupportInfo* info, const OrtNode* node) {
    info->groups.push_back({node});
    return nullptr;
}
const char* h_NodeComputeContext_NodeName(const OrtNodeComputeContext* c) { return c->name.c_str(); }
OrtStatus* h_EpDevice_AddAllocatorInfo(OrtEpDevice* d, const OrtMemoryInfo* info) {
    if (!d || !info) return mk(ORT_INVALID_ARGUMENT, "EpDevice_AddAllocatorInfo: null argument");
    d->allocator_infos.push_back(info);
    return nullptr;
}
const OrtMemoryDevice* h_MemoryInfo_GetMemoryDevice(const OrtMemoryInfo* m) { return &m->device; }
OrtMemoryInfoDeviceType h_MemoryDevice_GetDeviceType(const OrtMemoryDevice* d) { return d->type; }
uint32_t h_MemoryDevice_GetVendorId(const OrtMemoryDevice* d) { return d->vendor; }
uint32_t h_MemoryDevice_GetDeviceId(const OrtMemoryDevice* d) { return (uint32_t)d->id; }

// Function tables built from the shared slot lists.
void* g_api[ORTMI_ORT_API_TABLE_SIZE];
void* g_ep_api[ORTMI_ORT_EP_API_TABLE_SIZE];

#define CHECK_SIG(slot, name, ret, params) \
    static_assert(std::is_same<decltype(&h_##name), ort_abi::api::name##_fn>::value, #name);
#define CHECK_EP_SIG(slot, name, ret, params) \
    static_assert(std::is_same<decltype(&h_##name), ort_abi::ep_api::name##_fn>::value, #name);

const OrtEpApi* h_GetEpApi() { return reinterpret_cast<const OrtEpApi*>(g_ep_api); }

const OrtApi* get_api(uint32_t version) {
    static bool init = false;
    if (!init) {
#define FILL(slot, name, ret, params) g_api[slot] = reinterpret_cast<void*>(&h_##name);
#define FILL_EP(slot, name, ret, params) g_ep_api[slot] = reinterpret_cast<void*>(&h_##name);
        ORTMI_ORT_API_SLOTS(FILL)
        ORTMI_ORT_EP_API_SLOTS(FILL_EP)
#undef FILL
#undef FILL_EP
        init = true;
    }
    return version <= ORT_API_VERSION ? reinterpret_cast<const OrtApi*>(g_api) : nullptr;
}
const char* get_version_string() { return "1.29.0-harness"; }
OrtApiBase g_api_base{get_api, get_version_string};

}  // namespace

ORTMI_ORT_API_SLOTS(CHECK_SIG)
ORTMI_ORT_EP_API_SLOTS(CHECK_EP_SIG)

// The OrtEp slot the reference binds as
// fn(*const OrtEp, *mut *const OrtMemoryDevice) -> *mut OrtStatus (rust/src/ep.rs:104-113).
static_assert(std::is_same<decltype(OrtEp::GetDefaultMemoryDevice),
                           OrtStatus* (*)(const OrtEp*, const OrtMemoryDevice**)>::value,
              "OrtEp::GetDefaultMemoryDevice must return a status and take an out-parameter");

// ------------------------------------------------------------------ graph --
struct HxGraph {
    OrtGraph g;
    std::map<std::string, std::unique_ptr<OrtValueInfo>> values;
    std::vector<std::unique_ptr<OrtNode>> nodes;
    OrtValueInfo* value(const std::string& name) {
        auto it = values.find(name);
        if (it != values.end()) return it->second.get();
        auto v = std::make_unique<OrtValueInfo>();
        v->name = name;
        OrtValueInfo* p = v.get();
        values[name] = std::move(v);
        return p;
    }
};

// ---------------------------------------------------------------- session --
struct Partition {
    OrtGraph sub;
    OrtNode fused;
    OrtNodeComputeInfo* info = nullptr;
    void* state = nullptr;
};

struct DevBuf {
    void* ptr = nullptr;
    size_t bytes = 0;
};

// A value's copy on the EP's side of the placement rule (a fixed buffer per name,
// regrown only when a larger value comes).
struct Placed {
    OrtValue value;
    size_t bytes = 0;
};

struct Session {
    HxGraph* graph = nullptr;
    void* lib = nullptr;
    ReleaseEpFactoryFn release_factory = nullptr;
    OrtEpFactory* factory = nullptr;
    OrtEpDevice* ep_device = nullptr;
    OrtEp* ep = nullptr;
    OrtHardwareDevice gpu{OrtHardwareDeviceType_GPU}, cpu{OrtHardwareDeviceType_CPU};
    std::vector<std::unique_ptr<Partition>> parts;
    std::vector<std::unique_ptr<OrtValueInfo>> extra_vis;
    std::set<const OrtNode*> claimed;
    // Values of the current run (not owning), one persistent OrtValue per name
    // (owning: its fields are rewritten when the value is set again).
    std::unordered_map<std::string, OrtValue*> env;
    std::unordered_map<std::string, std::unique_ptr<OrtValue>> store;
    std::unordered_map<std::string, DevBuf> owned;              // harness-allocated outputs
    std::unordered_map<std::string, std::pair<void*, bool>> bound;  // caller-bound outputs (ptr, on device)
    // Placement rule state: the EP's default memory device (null: CPU memory), the
    // allocator the factory handed out for it, the EP's data transfer, the copies
    // of feeds and the staged outputs bound on the other side.
    const OrtMemoryDevice* ep_mem = nullptr;
    bool ep_dev = false;  // the EP's memory is GPU memory
    OrtAllocator* ep_alloc = nullptr;
    OrtDataTransferImpl* dt = nullptr;
    std::unordered_map<std::string, Placed> feeds, staged_outs;
    std::vector<std::pair<OrtValue*, std::string>> copy_back;  // staged output -> its binding
    int64_t copies = 0;                                        // data-transfer calls made by runs
    void* side_alloc(size_t bytes) {
        if (!ep_dev) return std::malloc(bytes ? bytes : 1);
        return ep_alloc ? ep_alloc->Alloc(ep_alloc, bytes ? bytes : 1) : nullptr;
    }
    void side_free(void* p) {
        if (!p) return;
        if (!ep_dev) std::free(p);
        else if (ep_alloc) ep_alloc->Free(ep_alloc, p);
    }
    OrtValue* value(const std::string& name) {
        auto& v = store[name];
        if (!v) v = std::make_unique<OrtValue>();
        return v.get();
    }
    std::vector<std::unique_ptr<OrtNodeComputeContext>> ctxs;
    ~Session();
};

static size_t esize(int dt) {
    switch (dt) {
        case 1: case 6: case 12: return 4;
        case 10: case 16: case 4: case 5: return 2;
        case 7: case 11: case 13: return 8;
        default: return 1;
    }
}

namespace {
OrtStatus* h_KernelContext_GetOutput(OrtKernelContext* c, size_t i, const int64_t* dims, size_t n,
                                     OrtValue** out) {
    if (i >= c->outputs.size()) return mk(ORT_INVALID_ARGUMENT, "output index out of range");
    Session* s = c->session;
    const std::string& name = c->outputs[i]->name;
    OrtValue* v = s->value(name);
    v->info.dims.assign(dims, dims + n);
    v->info.dtype = c->outputs[i]->type.dtype;
    size_t bytes = esize(v->info.dtype);
    for (size_t k = 0; k < n; ++k) bytes *= (size_t)(dims[k] < 0 ? 0 : dims[k]);
    auto b = s->bound.find(name);
    if (b != s->bound.end() && b->second.second == s->ep_dev) {
        v->data = b->second.first;  // bound on the EP's side: written in place
        v->on_device = s->ep_dev;
    } else if (b != s->bound.end()) {
        // Bound on the other side: produced in a buffer on the EP's side and copied
        // to the binding after Compute.
        Placed& st = s->staged_outs[name];
        if (st.bytes < bytes) {
            s->side_free(st.value.data);
            st.value.data = s->side_alloc(bytes);
            st.bytes = st.value.data ? bytes : 0;
            if (!st.value.data) return mk(ORT_FAIL, "harness: allocation failed for output " + name);
        }
        st.value.info = v->info;
        st.value.on_device = s->ep_dev;
        v->data = b->second.first;
        v->on_device = b->second.second;
        s->copy_back.push_back({&st.value, name});
        *out = &st.value;
        s->env[name] = v;
        return nullptr;
    } else {
        // Nobody binds it: allocated on the EP's side.
        DevBuf& buf = s->owned[name];
        if (buf.bytes < bytes) {
            s->side_free(buf.ptr);
            buf.ptr = s->side_alloc(bytes);
            buf.bytes = buf.ptr ? bytes : 0;
            if (!buf.ptr) return mk(ORT_FAIL, "harness: allocation failed for output " + name);
        }
        v->data = buf.ptr;
        v->on_device = s->ep_dev;
    }
    *out = v;
    s->env[name] = v;
    return nullptr;
}
}  // namespace

Session::~Session() {
    for (auto& p : parts)
        if (p->info && p->info->ReleaseState) p->info->ReleaseState(p->info, p->state);
    if (ep && !parts.empty()) {
        std::vector<OrtNodeComputeInfo*> infos;
        for (auto& p : parts) infos.push_back(p->info);
        ep->ReleaseNodeComputeInfos(ep, infos.data(), infos.size());
    }
    for (auto& kv : owned) side_free(kv.second.ptr);
    for (auto* m : {&feeds, &staged_outs})
        for (auto& kv : *m) side_free(kv.second.value.data);
    if (ep_alloc) factory->ReleaseAllocator(factory, ep_alloc);
    if (dt) dt->Release(dt);
    if (ep) factory->ReleaseEp(factory, ep);
    if (ep_device) h_ReleaseEpDevice(ep_device);
    if (factory && release_factory) release_factory(factory);
    if (lib) dlclose(lib);
}

static bool take(OrtStatus* st, const char* what) {
    if (!st) return true;
    g_err = std::string(what) + ": " + st->msg;
    delete st;
    return false;
}

extern "C" {

const char* hx_last_error() { return g_err.c_str(); }
const OrtApiBase* hx_api_base() { return &g_api_base; }

HxGraph* hx_graph_new() { return new HxGraph(); }
void hx_graph_free(HxGraph* g) { delete g; }

int hx_graph_add_value(HxGraph* g, const char* name, int dtype, int rank, const int64_t* dims) {
    OrtValueInfo* v = g->value(name);
    v->type.dtype = dtype;
    v->type.dims.assign(dims, dims + rank);
    return 0;
}

int hx_graph_add_initializer(HxGraph* g, const char* name, int dtype, int rank,
                             const int64_t* dims, const void* data, size_t nbytes) {
    OrtValueInfo* v = g->value(name);
    v->type.dtype = dtype;
    v->type.dims.assign(dims, dims + rank);
    v->is_initializer = true;
    v->init.info = v->type;
    v->init.host.assign((const uint8_t*)data, (const uint8_t*)data + nbytes);
    v->init.data = v->init.host.data();
    g->g.initializers.push_back(v);
    return 0;
}

int hx_graph_add_node(HxGraph* g, const char* op, const char* domain, const char* name, int since,
                      int n_in, const char** inputs, int n_out, const char** outputs) {
    auto n = std::make_unique<OrtNode>();
    n->id = g->nodes.size();
    n->op = op;
    n->domain = domain ? domain : "";
    n->name = name ? name : "";
    n->since = since;
    for (int i = 0; i < n_in; ++i)
        n->inputs.push_back(inputs[i] && *inputs[i] ? g->value(inputs[i]) : nullptr);
    for (int i = 0; i < n_out; ++i) {
        OrtValueInfo* v = outputs[i] && *outputs[i] ? g->value(outputs[i]) : nullptr;
        if (v) {
            v->producer = n.get();
            v->producer_output = i;
        }
        n->outputs.push_back(v);
    }
    g->g.nodes.push_back(n.get());
    g->nodes.push_back(std::move(n));
    return (int)g->nodes.size() - 1;
}

static OrtOpAttr* new_attr(HxGraph* g, int node, const char* name, OrtOpAttrType t) {
    auto a = std::make_unique<OrtOpAttr>();
    a->name = name;
    a->type = t;
    OrtOpAttr* p = a.get();
    g->nodes[node]->attrs.push_back(std::move(a));
    return p;
}
int hx_node_attr_int(HxGraph* g, int node, const char* name, int64_t v) {
    new_attr(g, node, name, ORT_OP_ATTR_INT)->i = v;
    return 0;
}
int hx_node_attr_float(HxGraph* g, int node, const char* name, float v) {
    new_attr(g, node, name, ORT_OP_ATTR_FLOAT)->f = v;
    return 0;
}
int hx_node_attr_string(HxGraph* g, int node, const char* name, const char* v) {
    new_attr(g, node, name, ORT_OP_ATTR_STRING)->s = v;
    return 0;
}
int hx_node_attr_ints(HxGraph* g, int node, const char* name, int n, const int64_t* v) {
    new_attr(g, node, name, ORT_OP_ATTR_INTS)->ints.assign(v, v + n);
    return 0;
}

int hx_graph_set_metadata(HxGraph* g, const char* key, const char* value) {
    g->g.metadata[key] = value;
    return 0;
}

int hx_graph_set_io(HxGraph* g, int n_in, const char** ins, int n_out, const char** outs) {
    g->g.inputs.clear();
    g->g.outputs.clear();
    for (int i = 0; i < n_in; ++i) g->g.inputs.push_back(g->value(ins[i]));
    for (int i = 0; i < n_out; ++i) g->g.outputs.push_back(g->value(outs[i]));
    return 0;
}

// Load the EP, run device selection, CreateEp and GetCapability. With
// compile = 0 the session stops after GetCapability (no GPU work at all).
// force_device = 1 creates the EP on the GPU hardware device even when the EP
// offered none (no GPU visible): only GetCapability runs then, for CPU tests of
// the claim and partition logic.
Session* hx_session_new(HxGraph* g, const char* ep_path, const char* registration_name,
                        int compile, int force_device) {
    auto s = std::make_unique<Session>();
    s->graph = g;
    s->lib = dlopen(ep_path, RTLD_NOW | RTLD_LOCAL);
    if (!s->lib) {
        g_err = std::string("dlopen: ") + dlerror();
        return nullptr;
    }
    auto create = (CreateEpFactoriesFn)dlsym(s->lib, "CreateEpFactories");
    s->release_factory = (ReleaseEpFactoryFn)dlsym(s->lib, "ReleaseEpFactory");
    if (!create || !s->release_factory) {
        g_err = "EP library lacks CreateEpFactories / ReleaseEpFactory";
        return nullptr;
    }
    OrtEpFactory* facs[4] = {};
    size_t nf = 0;
    if (!take(create(registration_name, &g_api_base, nullptr, facs, 4, &nf), "CreateEpFactories"))
        return nullptr;
    if (nf < 1) {
        g_err = "no factory";
        return nullptr;
    }
    s->factory = facs[0];
    const OrtHardwareDevice* hw[2] = {&s->cpu, &s->gpu};
    OrtEpDevice* devs[2] = {};
    size_t nd = 0;
    if (!take(s->factory->GetSupportedDevices(s->factory, hw, 2, devs, 2, &nd), "GetSupportedDevices"))
        return nullptr;
    const OrtHardwareDevice* sel[1] = {&s->gpu};
    if (nd >= 1) {
        s->ep_device = devs[0];
        sel[0] = s->ep_device->device;
    } else if (!force_device || compile) {
        g_err = "EP offered no device (is a GPU visible?)";
        return nullptr;
    }
    if (!take(s->factory->CreateEp(s->factory, sel, nullptr, 1, nullptr, nullptr, &s->ep), "CreateEp"))
        return nullptr;
    OrtEpGraphSupportInfo support;
    if (!take(s->ep->GetCapability(s->ep, &g->g, &support), "GetCapability")) return nullptr;
    for (auto& grp : support.groups) {
        auto p = std::make_unique<Partition>();
        std::set<const OrtNode*> in_group(grp.begin(), grp.end());
        for (const OrtNode* n : grp) s->claimed.insert(n);
        std::set<std::string> produced, consumed_outside;
        for (auto& n : g->nodes)
            if (!in_group.count(n.get()))
                for (auto* v : n->inputs)
                    if (v) consumed_outside.insert(v->name);
        for (auto* v : g->g.outputs) consumed_outside.insert(v->name);
        std::vector<std::string> ins, outs;
        std::set<std::string> seen_in;
        for (const OrtNode* n : grp) {
            p->sub.nodes.push_back(const_cast<OrtNode*>(n));
            for (auto* v : n->outputs)
                if (v) produced.insert(v->name);
        }
        std::set<std::string> seen_init;
        for (const OrtNode* n : grp) {
            for (auto* v : n->inputs) {
                if (!v || produced.count(v->name)) continue;
                if (v->is_initializer) {  // constants are dropped from the fused inputs
                    if (seen_init.insert(v->name).second) p->sub.initializers.push_back(v);
                    continue;
                }
                if (seen_in.insert(v->name).second) {
                    ins.push_back(v->name);
                    p->fused.inputs.push_back(v);
                    p->sub.inputs.push_back(v);
                }
            }
            for (auto* v : n->outputs)
                if (v && consumed_outside.count(v->name)) {
                    outs.push_back(v->name);
                    p->fused.outputs.push_back(v);
                    p->sub.outputs.push_back(v);
                }
        }
        p->fused.name = "MI355X_fused_" + std::to_string(s->parts.size());
        p->fused.op = p->fused.name;
        p->fused.domain = "";
        s->parts.push_back(std::move(p));
    }
    if (!compile) return s.release();
    for (auto& n : g->nodes)
        if (!s->claimed.count(n.get())) {
            g_err = "node " + n->name + " (" + n->op + ") was not claimed and the harness has no "
                    "CPU execution provider";
            return nullptr;
        }
    std::vector<const OrtGraph*> graphs;
    std::vector<const OrtNode*> fused;
    for (auto& p : s->parts) {
        graphs.push_back(&p->sub);
        fused.push_back(&p->fused);
    }
    // Placement: the EP's default memory device, and for a GPU one the allocator the
    // factory hands out for the matching memory info the EP device registered (as
    // ORT creates the device allocators of a session); the EP's data transfer.
    if (!s->ep->GetDefaultMemoryDevice) {
        g_err = "OrtEp::GetDefaultMemoryDevice is not set";
        return nullptr;
    }
    if (!take(s->ep->GetDefaultMemoryDevice(s->ep, &s->ep_mem), "GetDefaultMemoryDevice"))
        return nullptr;
    s->ep_dev = s->ep_mem && s->ep_mem->type != OrtMemoryInfoDeviceType_CPU;
    if (s->ep_dev) {
        const OrtMemoryInfo* info = nullptr;
        if (s->ep_device)
            for (const OrtMemoryInfo* m : s->ep_device->allocator_infos)
                if (&m->device == s->ep_mem) info = m;
        if (!info) {
            g_err = "the EP's default memory device is not one its EP device registered";
            return nullptr;
        }
        if (!take(s->factory->CreateAllocator(s->factory, info, nullptr, &s->ep_alloc),
                  "CreateAllocator"))
            return nullptr;
        if (!s->ep_alloc) {
            g_err = "the EP factory gave no allocator for its own memory info";
            return nullptr;
        }
    }
    if (!take(s->factory->CreateDataTransfer(s->factory, &s->dt), "CreateDataTransfer"))
        return nullptr;
    if (!s->dt || !s->dt->CopyTensors || !s->dt->CanCopy || !s->dt->Release) {
        g_err = "CreateDataTransfer returned an incomplete OrtDataTransferImpl";
        return nullptr;
    }
    std::vector<OrtNodeComputeInfo*> infos(s->parts.size(), nullptr);
    std::vector<OrtNode*> ctx_nodes(s->parts.size(), nullptr);
    if (!take(s->ep->Compile(s->ep, graphs.data(), fused.data(), graphs.size(), infos.data(),
                             ctx_nodes.data()),
              "Compile"))
        return nullptr;
    for (size_t i = 0; i < s->parts.size(); ++i) {
        s->parts[i]->info = infos[i];
        auto ctx = std::make_unique<OrtNodeComputeContext>();
        ctx->name = s->parts[i]->fused.name;
        if (!take(infos[i]->CreateState(infos[i], ctx.get(), &s->parts[i]->state), "CreateState"))
            return nullptr;
        s->ctxs.push_back(std::move(ctx));
    }
    return s.release();
}

void hx_session_free(Session* s) { delete s; }

int hx_session_num_partitions(Session* s) { return (int)s->parts.size(); }
int hx_session_partition_size(Session* s, int i) { return (int)s->parts[i]->sub.nodes.size(); }
int hx_session_partition_node(Session* s, int i, int j) { return (int)s->parts[i]->sub.nodes[j]->id; }
int hx_session_node_claimed(Session* s, int node) {
    return s->claimed.count(s->graph->nodes[node].get()) ? 1 : 0;
}

// Bind a caller-owned device buffer as the storage of a graph value produced by
// the EP (an IOBinding analogue; binding a present-KV output to the past-KV input
// buffer gives the shared-buffer contract).
static bool is_device_memory(const void* p) {
    hipPointerAttribute_t attr;
    if (!p || hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeDevice || attr.type == hipMemoryTypeManaged;
}

int hx_session_bind_output(Session* s, const char* name, void* ptr) {
    if (ptr) s->bound[name] = {ptr, is_device_memory(ptr)};
    else s->bound.erase(name);
    return 0;
}

int hx_session_set_input(Session* s, const char* name, void* ptr, int dtype, int rank,
                         const int64_t* dims) {
    OrtValue* v = s->value(name);
    if (v->data != ptr || !ptr) v->on_device = is_device_memory(ptr);  // classified once per buffer
    v->data = ptr;
    v->info.dtype = dtype;
    v->info.dims.assign(dims, dims + rank);
    s->env[name] = v;
    return 0;
}

int hx_session_run(Session* s) {
    // Run partitions in dependency order: a partition is ready once every fused
    // input is available (a graph input or an output of a finished partition).
    // Values produced by partitions are dropped first, so a partition never runs on
    // a previous run's outputs.
    for (auto& p : s->parts)
        for (auto* v : p->fused.outputs) s->env.erase(v->name);
    std::vector<bool> done(s->parts.size(), false);
    for (size_t round = 0; round < s->parts.size(); ++round) {
        bool progressed = false;
        for (size_t pi = 0; pi < s->parts.size(); ++pi) {
            if (done[pi]) continue;
            auto& p = s->parts[pi];
            bool ready = true;
            for (auto* v : p->fused.inputs)
                if (!s->env.count(v->name)) ready = false;
            if (!ready) continue;
            OrtKernelContext ctx;
            ctx.session = s;
            ctx.inputs.reserve(p->fused.inputs.size());
            // Feeds on the other side of the EP's memory are copied over first, in one
            // data-transfer call.
            std::vector<const OrtValue*> srcs;
            std::vector<OrtValue*> dsts;
            for (auto* vi : p->fused.inputs) {
                OrtValue* v = s->env[vi->name];
                if (v->on_device != s->ep_dev) {
                    Placed& st = s->feeds[vi->name];
                    size_t bytes = esize(v->info.dtype);
                    for (int64_t d : v->info.dims) bytes *= (size_t)(d < 0 ? 0 : d);
                    if (st.bytes < bytes) {
                        s->side_free(st.value.data);
                        st.value.data = s->side_alloc(bytes);
                        st.bytes = st.value.data ? bytes : 0;
                        if (!st.value.data) {
                            g_err = "harness: allocation failed for feed " + vi->name;
                            return 1;
                        }
                    }
                    st.value.info = v->info;
                    st.value.on_device = s->ep_dev;
                    srcs.push_back(v);
                    dsts.push_back(&st.value);
                    v = &st.value;
                }
                ctx.inputs.push_back(v);
            }
            if (!srcs.empty()) {
                // Host memory is a null device; device memory the EP did not declare
                // is GPU 0 of AMD's vendor id.
                static const OrtMemoryDevice gpu0{OrtMemoryInfoDeviceType_GPU, 0x1002, 0, {}};
                const OrtMemoryDevice* src_dev = s->ep_dev ? nullptr : &gpu0;
                const OrtMemoryDevice* dst_dev = s->ep_dev ? s->ep_mem : nullptr;
                if (!s->dt->CanCopy(s->dt, src_dev, dst_dev)) {
                    g_err = "the EP's data transfer cannot copy feeds to its memory device";
                    return 1;
                }
                ++s->copies;
                if (!take(s->dt->CopyTensors(s->dt, srcs.data(), dsts.data(), nullptr, srcs.size()),
                          "CopyTensors (feeds)"))
                    return 1;
            }
            ctx.outputs.assign(p->fused.outputs.begin(), p->fused.outputs.end());
            s->copy_back.clear();
            if (!take(p->info->Compute(p->info, p->state, &ctx), "Compute")) return 1;
            // Outputs bound on the other side: staged on the EP's side, copied back.
            if (!s->copy_back.empty()) {
                std::vector<const OrtValue*> from;
                std::vector<OrtValue*> to;
                for (auto& cb : s->copy_back) {
                    from.push_back(cb.first);
                    to.push_back(s->env[cb.second]);
                }
                ++s->copies;
                if (!take(s->dt->CopyTensors(s->dt, from.data(), to.data(), nullptr, from.size()),
                          "CopyTensors (outputs)"))
                    return 1;
                s->copy_back.clear();
            }
            done[pi] = progressed = true;
        }
        if (!progressed) break;
    }
    for (size_t pi = 0; pi < s->parts.size(); ++pi)
        if (!done[pi]) {
            g_err = "partition " + std::to_string(pi) + " never became ready (missing input)";
            return 1;
        }
    return 0;
}

// Data-transfer calls the placement rule made so far (feeds in, outputs back).
int64_t hx_session_copies(Session* s) { return s->copies; }

// The EP's default memory device as the session placed values: type
// (OrtMemoryInfoDeviceType; CPU when the EP reports null), vendor id, device id.
int hx_session_memory_device(Session* s, int* type, uint32_t* vendor, int* id) {
    *type = s->ep_mem ? (int)s->ep_mem->type : (int)OrtMemoryInfoDeviceType_CPU;
    *vendor = s->ep_mem ? s->ep_mem->vendor : 0;
    *id = s->ep_mem ? s->ep_mem->id : 0;
    return 0;
}

// OrtEp::GetDefaultMemoryDevice: 0 on success with *is_cpu = 1 when the EP
// reports CPU memory (a null OrtMemoryDevice).
int hx_session_default_memory_device(Session* s, int* is_cpu) {
    const OrtMemoryDevice* dev = reinterpret_cast<const OrtMemoryDevice*>(&g_err);  // poison
    if (!s->ep->GetDefaultMemoryDevice) {
        g_err = "GetDefaultMemoryDevice is not set";
        return 1;
    }
    if (!take(s->ep->GetDefaultMemoryDevice(s->ep, &dev), "GetDefaultMemoryDevice")) return 1;
    *is_cpu = (dev == nullptr || dev->type == OrtMemoryInfoDeviceType_CPU) ? 1 : 0;
    return 0;
}

// OrtEpFactory::CreateAllocator for a memory info (name, id), as ORT calls it for
// the memory infos an EP device registers. Returns -1 on error, 0 when the EP
// hands out no allocator, 1 when it does: then the allocator is exercised (Info,
// Alloc of `bytes` device bytes checked by a fill and copy-back, Reserve, Free)
// and released through ReleaseAllocator.
int hx_factory_allocator_check(Session* s, const char* mem_name, int id, size_t bytes) {
    OrtMemoryInfo* info = nullptr;
    if (!take(h_CreateMemoryInfo(mem_name, OrtDeviceAllocator, id, OrtMemTypeDefault, &info),
              "CreateMemoryInfo"))
        return -1;
    std::unique_ptr<OrtMemoryInfo> hold(info);
    OrtAllocator* a = reinterpret_cast<OrtAllocator*>(&g_err);  // poison: the EP must write it
    if (!take(s->factory->CreateAllocator(s->factory, info, nullptr, &a), "CreateAllocator"))
        return -1;
    if (!a) return 0;
    auto fail_with = [&](const std::string& m) {
        g_err = m;
        s->factory->ReleaseAllocator(s->factory, a);
        return -1;
    };
    if (a->version < 18 || !a->Alloc || !a->Free || !a->Info)
        return fail_with("allocator lacks Alloc/Free/Info or reports version < 18");
    if (a->Info(a) != info) return fail_with("allocator Info() is not the memory info it was made for");
    void* p = a->Alloc(a, bytes);
    if (!p) return fail_with("Alloc returned null");
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, p) != hipSuccess || attr.type != hipMemoryTypeDevice ||
        attr.device != id) {
        (void)hipGetLastError();
        a->Free(a, p);
        return fail_with("Alloc did not return device memory of GPU " + std::to_string(id));
    }
    std::vector<uint8_t> back(bytes, 0);
    bool ok = hipMemset(p, 0x5A, bytes) == hipSuccess &&
              hipMemcpy(back.data(), p, bytes, hipMemcpyDeviceToHost) == hipSuccess;
    for (size_t i = 0; ok && i < bytes; ++i) ok = back[i] == 0x5A;
    a->Free(a, p);
    if (!ok) return fail_with("allocated memory did not hold a fill pattern");
    if (a->Reserve) {
        void* r = a->Reserve(a, bytes);
        if (!r) return fail_with("Reserve returned null");
        a->Free(a, r);
    }
    s->factory->ReleaseAllocator(s->factory, a);
    return 1;
}

// OrtEpFactory::CreateDataTransfer + CanCopy + CopyTensors of one tensor
// (src and dst host or device pointers of the same dtype and shape), then Release.
int hx_factory_data_transfer_copy(Session* s, void* src, void* dst, int dtype, int rank,
                                  const int64_t* dims) {
    OrtDataTransferImpl* dt = nullptr;
    if (!take(s->factory->CreateDataTransfer(s->factory, &dt), "CreateDataTransfer")) return 1;
    if (!dt || !dt->CopyTensors || !dt->Release || !dt->CanCopy) {
        g_err = "CreateDataTransfer returned an incomplete OrtDataTransferImpl";
        return 1;
    }
    if (!dt->CanCopy(dt, nullptr, nullptr)) {
        dt->Release(dt);
        g_err = "CanCopy refused a CPU <-> CPU copy";
        return 1;
    }
    OrtValue a, b;
    a.data = src;
    b.data = dst;
    a.info.dtype = b.info.dtype = dtype;
    a.info.dims.assign(dims, dims + rank);
    b.info.dims = a.info.dims;
    const OrtValue* srcs[1] = {&a};
    OrtValue* dsts[1] = {&b};
    const bool ok = take(dt->CopyTensors(dt, srcs, dsts, nullptr, 1), "CopyTensors");
    dt->Release(dt);
    return ok ? 0 : 1;
}

int hx_session_get_output(Session* s, const char* name, void** ptr, int* rank, int64_t* dims) {
    auto it = s->env.find(name);
    if (it == s->env.end()) {
        g_err = std::string("no value ") + name;
        return 1;
    }
    *ptr = it->second->data;
    *rank = (int)it->second->info.dims.size();
    for (int i = 0; i < *rank && i < 8; ++i) dims[i] = it->second->info.dims[i];
    return 0;
}

}  // extern "C"
