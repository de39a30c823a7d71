// C-ABI surface of the MI355X plugin execution provider: CreateEpFactories /
// ReleaseEpFactory and the OrtEpFactory / OrtEp / OrtNodeComputeInfo vtables.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <set>

#include "../../../include/ortmi_kernels.h"
#include "ep_internal.h"

#define ORTMI_EXPORT extern "C" __attribute__((visibility("default")))

namespace ortmi_ep {

using namespace ort_abi;

namespace {

constexpr uint32_t kVendorIdAmd = 0x1002;
constexpr const char* kDefaultName = "MI355XExecutionProvider";
constexpr const char* kVersion = "0.29.0";

// Nothing may unwind across the ABI (rust/src/lib.rs:37-71): every entry runs
// its body under this guard and turns exceptions into an OrtStatus.
template <typename F>
OrtStatus* guard(const OrtApi* a, const char* what, F&& body) {
    try {
        body();
        return nullptr;
    } catch (const EpError& e) {
        std::string m = std::string("MI355X EP ") + what + ": " + e.what();
        return a ? api::CreateStatus(a)(e.code, m.c_str()) : nullptr;
    } catch (const std::exception& e) {
        std::string m = std::string("MI355X EP ") + what + ": " + e.what();
        return a ? api::CreateStatus(a)(ORT_EP_FAIL, m.c_str()) : nullptr;
    } catch (...) {
        std::string m = std::string("MI355X EP ") + what + ": unknown failure";
        return a ? api::CreateStatus(a)(ORT_EP_FAIL, m.c_str()) : nullptr;
    }
}

bool env_flag(const char* name) {
    const char* v = std::getenv(name);
    return v && *v && std::strcmp(v, "0") != 0;
}

// ------------------------------------------------------------- allocator --
// Name of the memory info whose allocator this EP hands out: HBM of the GPU
// given by the memory info's id. Any other memory info gets no allocator (a null
// OrtAllocator and a null status, the reference's answer for every memory info,
// rust/src/factory.rs:221-235), so ORT keeps using its own.
constexpr const char* kHbmMemoryInfoName = "MI355X_HBM";

struct DeviceAllocator {
    OrtAllocator base;  // first member: an OrtAllocator* is a DeviceAllocator*
    const OrtMemoryInfo* info;
    int device;
};

// Runs `body` with `device` current and restores the caller's current device.
template <typename F>
bool on_device(int device, F&& body) {
    int prev = -1;
    if (hipGetDevice(&prev) != hipSuccess) prev = -1;
    if (prev != device && hipSetDevice(device) != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    const bool ok = body();
    if (prev >= 0 && prev != device) (void)hipSetDevice(prev);
    return ok;
}

void* alloc_fn(OrtAllocator* self, size_t size) {
    auto* d = reinterpret_cast<DeviceAllocator*>(self);
    void* p = nullptr;
    on_device(d->device, [&] {
        if (hipMalloc(&p, size ? size : 1) == hipSuccess) return true;
        (void)hipGetLastError();
        p = nullptr;
        return false;
    });
    return p;
}
void free_fn(OrtAllocator* self, void* p) {
    if (!p) return;
    auto* d = reinterpret_cast<DeviceAllocator*>(self);
    on_device(d->device, [&] { return hipFree(p) == hipSuccess; });
}
const OrtMemoryInfo* info_fn(const OrtAllocator* self) {
    return reinterpret_cast<const DeviceAllocator*>(self)->info;
}
void* reserve_fn(OrtAllocator* self, size_t size) { return alloc_fn(self, size); }
void* alloc_on_stream_fn(OrtAllocator* self, size_t size, OrtSyncStreamImpl*) {
    return alloc_fn(self, size);
}

// --------------------------------------------------------- data transfer --
struct DataTransfer {
    OrtDataTransferImpl base;
    const OrtApi* api;
    const OrtEpApi* ep_api;
    hipStream_t stream = nullptr;  // copies of one CopyTensors call, then one synchronisation
    // Pinned staging for small device-to-host copies into pageable memory: 12.7
    // against 20.4 us for 8 bytes (the DMA engine reads pinned memory directly).
    char* pinned = nullptr;
    size_t pinned_bytes = 0;
};
constexpr size_t kPinnedStageMax = 1 << 20;

void dt_release(OrtDataTransferImpl* self) {
    auto* t = reinterpret_cast<DataTransfer*>(self);
    if (t->stream) (void)hipStreamDestroy(t->stream);
    if (t->pinned) (void)hipHostFree(t->pinned);
    delete t;
}
// Host memory, or memory of an AMD GPU: hipMemcpyDefault copies between any two
// of them (unified addressing). A null memory device is host memory.
bool dt_side_ok(const DataTransfer* t, const OrtMemoryDevice* d) {
    if (!d) return true;
    const OrtMemoryInfoDeviceType ty = ep_api::MemoryDevice_GetDeviceType(t->ep_api)(d);
    if (ty == OrtMemoryInfoDeviceType_CPU) return true;
    return ty == OrtMemoryInfoDeviceType_GPU &&
           ep_api::MemoryDevice_GetVendorId(t->ep_api)(d) == kVendorIdAmd;
}
bool dt_can_copy(const OrtDataTransferImpl* self, const OrtMemoryDevice* src,
                 const OrtMemoryDevice* dst) {
    const auto* t = reinterpret_cast<const DataTransfer*>(self);
    return dt_side_ok(t, src) && dt_side_ok(t, dst);
}
// Where a pointer lives: 0 host memory the runtime does not know (pageable), 1
// pinned host memory, 2 device memory (a query of about 0.5 us).
int mem_kind(const void* p) {
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();  // the query's error must not reach the next launch check
        return 0;
    }
    if (attr.type == hipMemoryTypeDevice) return 2;
    return attr.type == hipMemoryTypeHost ? 1 : -1;
}
OrtStatus* dt_copy(OrtDataTransferImpl* self, const OrtValue** src, OrtValue** dst,
                   OrtSyncStreamImpl**, size_t n) {
    auto* t = reinterpret_cast<DataTransfer*>(self);
    const OrtApi* a = t->api;
    return guard(a, "CopyTensors", [&] {
        if (!t->stream)
            check_hip(hipStreamCreateWithFlags(&t->stream, hipStreamNonBlocking), "hipStreamCreate");
        struct Copy {
            const void* s;
            void* d;
            size_t bytes;
            int ks, kd;  // mem_kind of source and destination
        };
        std::vector<Copy> cs(n);
        size_t total = 0;
        for (size_t i = 0; i < n; ++i) {
            OrtTensorTypeAndShapeInfo* info = nullptr;
            check_ort(a, api::GetTensorTypeAndShape(a)(src[i], &info), "GetTensorTypeAndShape");
            size_t count = 0;
            ONNXTensorElementDataType et = ONNX_TENSOR_ELEMENT_DATA_TYPE_UNDEFINED;
            OrtStatus* s1 = api::GetTensorShapeElementCount(a)(info, &count);
            OrtStatus* s2 = s1 ? nullptr : api::GetTensorElementType(a)(info, &et);
            api::ReleaseTensorTypeAndShapeInfo(a)(info);
            check_ort(a, s1, "GetTensorShapeElementCount");
            check_ort(a, s2, "GetTensorElementType");
            Copy& c = cs[i];
            check_ort(a, api::GetTensorData(a)(src[i], &c.s), "GetTensorData");
            check_ort(a, api::GetTensorMutableData(a)(dst[i], &c.d), "GetTensorMutableData");
            c.bytes = count * dtype_size(et);
            c.ks = c.bytes ? mem_kind(c.s) : 0;
            c.kd = c.bytes ? mem_kind(c.d) : 2;
            total += c.bytes;
        }
        // A few small host-to-device copies (a decode step's input ids and length
        // scalars) go in one launch that carries the bytes (ortmi_copy_small_h2d):
        // 12.7 against 21.5 us for three 8-byte DMA copies and their synchronisation.
        bool small = n > 0 && n <= (size_t)ORTMI_SMALL_COPIES &&
                     total <= (size_t)ORTMI_SMALL_COPY_BYTES;
        for (const Copy& c : cs)
            if (c.bytes && !((c.ks == 0 || c.ks == 1) && c.kd == 2)) small = false;
        if (small) {
            std::vector<void*> sd;
            std::vector<const void*> ss;
            std::vector<size_t> sb;
            for (const Copy& c : cs) {
                sd.push_back(c.d);
                ss.push_back(c.s);
                sb.push_back(c.bytes);
            }
            check_kernel(ortmi_copy_small_h2d((int)n, sd.data(), ss.data(), sb.data(), t->stream),
                         "small copy");
            check_hip(hipStreamSynchronize(t->stream), "hipStreamSynchronize");
            return;
        }
        // Device-to-pageable-host copies of up to 1 MiB in all land in the pinned
        // staging buffer first and are copied out on the host after the
        // synchronisation.
        size_t staged = 0;
        for (const Copy& c : cs)
            if (c.bytes && c.ks == 2 && c.kd == 0) staged += (c.bytes + 255) & ~(size_t)255;
        const bool stage = staged && staged <= kPinnedStageMax;
        if (stage && t->pinned_bytes < staged) {
            if (t->pinned) check_hip(hipHostFree(t->pinned), "hipHostFree");
            t->pinned = nullptr;
            t->pinned_bytes = 0;
            check_hip(hipHostMalloc((void**)&t->pinned, kPinnedStageMax, hipHostMallocDefault),
                      "hipHostMalloc");
            t->pinned_bytes = kPinnedStageMax;
        }
        std::vector<std::pair<size_t, size_t>> outs;  // (copy index, staging offset)
        size_t off = 0;
        for (size_t i = 0; i < n; ++i) {
            const Copy& c = cs[i];
            if (!c.bytes) continue;
            if (stage && c.ks == 2 && c.kd == 0) {
                check_hip(hipMemcpyAsync(t->pinned + off, c.s, c.bytes, hipMemcpyDeviceToHost,
                                         t->stream),
                          "hipMemcpyAsync");
                outs.emplace_back(i, off);
                off += (c.bytes + 255) & ~(size_t)255;
            } else {
                check_hip(hipMemcpyAsync(c.d, c.s, c.bytes, hipMemcpyDefault, t->stream),
                          "hipMemcpyAsync");
            }
        }
        check_hip(hipStreamSynchronize(t->stream), "hipStreamSynchronize");
        for (const auto& o : outs) std::memcpy(cs[o.first].d, t->pinned + o.second, cs[o.first].bytes);
    });
}

// -------------------------------------------------------- compute info --
struct ComputeInfo {
    OrtNodeComputeInfo base;
    const OrtApi* api;
    std::unique_ptr<Plan> plan;
    std::string name;
};

OrtStatus* ci_create_state(OrtNodeComputeInfo* self, OrtNodeComputeContext*, void** state) {
    // The plan is the state (rust/src/ep.rs:1918-1927).
    *state = self;
    return nullptr;
}
OrtStatus* ci_compute(OrtNodeComputeInfo* self, void* state, OrtKernelContext* ctx) {
    auto* ci = reinterpret_cast<ComputeInfo*>(state ? state : self);
    return guard(ci->api, "Compute", [&] { ci->plan->compute(ci->api, ctx); });
}
void ci_release_state(OrtNodeComputeInfo*, void*) {}

// --------------------------------------------------------------------- EP --
struct Factory;

struct Ep {
    OrtEp base;
    Factory* factory;
    const OrtApi* api;
    const OrtEpApi* ep_api;
    std::string name;
    int device = 0;
    const OrtMemoryDevice* memory_device = nullptr;  // null: CPU memory
};

struct Factory {
    OrtEpFactory base;
    const OrtApi* api;
    const OrtEpApi* ep_api;
    std::string name, vendor, version;
    // HBM of GPU 0, registered on the EP device as its allocator's memory info:
    // ORT allocates the fused nodes' inputs and outputs there and copies host
    // values in and out through CreateDataTransfer. Owned by the factory.
    OrtMemoryInfo* hbm_info = nullptr;
    ~Factory() {
        if (hbm_info) api::ReleaseMemoryInfo(api)(hbm_info);
    }
};

const char* ep_get_name(const OrtEp* self) { return reinterpret_cast<const Ep*>(self)->name.c_str(); }

// Value of one entry of the model's custom metadata map; false when absent.
bool read_metadata(const OrtApi* a, const OrtGraph* graph, const char* key, std::string* value) {
    OrtModelMetadata* md = nullptr;
    check_ort(a, api::Graph_GetModelMetadata(a)(graph, &md), "Graph_GetModelMetadata");
    OrtAllocator* alloc = nullptr;
    char* v = nullptr;
    OrtStatus* st = api::GetAllocatorWithDefaultOptions(a)(&alloc);
    if (!st) st = api::ModelMetadataLookupCustomMetadataMap(a)(md, alloc, key, &v);
    api::ReleaseModelMetadata(a)(md);
    check_ort(a, st, "ModelMetadataLookupCustomMetadataMap");
    if (!v) return false;
    *value = v;
    alloc->Free(alloc, v);
    return true;
}

OrtStatus* ep_get_capability(OrtEp* self, const OrtGraph* graph, OrtEpGraphSupportInfo* support) {
    Ep* ep = reinterpret_cast<Ep*>(self);
    return guard(ep->api, "GetCapability", [&] {
        GraphIR g = read_graph(ep->api, graph);
        std::vector<bool> claimed(g.nodes.size(), false);
        const bool debug = env_flag("ORTMI_EP_CLAIM_DEBUG");
        for (size_t i = 0; i < g.nodes.size(); ++i) {
            std::string why = claim_reason(g.nodes[i], g);
            claimed[i] = why.empty();
            if (debug && !why.empty())
                std::fprintf(stderr, "[mi355x-ep] decline %s (%s): %s\n", g.nodes[i].name.c_str(),
                             g.nodes[i].op.c_str(), why.c_str());
        }
        auto clusters = build_clusters(g, claimed);
        // Layer groups of large decoders (rust/src/ep.rs:296-332): boundaries from
        // the model metadata, else inferred; none inside a control-flow body.
        const OrtNode* parent = nullptr;
        check_ort(ep->api, api::Graph_GetParentNode(ep->api)(graph, &parent), "Graph_GetParentNode");
        const char* env = std::getenv("ONNXRUNTIME_EP_MLX_LAYER_PARTITIONS");
        const size_t span = parent ? 0 : select_layer_span(env);
        if (span) {
            std::set<std::string> bounds;
            std::string md;
            if (read_metadata(ep->api, graph, kLayerBoundaryKey, &md)) {
                std::vector<std::string> names;
                if (parse_json_string_array(md, &names)) {
                    for (auto& n : names)
                        if (!n.empty()) bounds.insert(n);
                } else {
                    std::fprintf(stderr, "[mi355x-ep] ignoring invalid %s metadata\n",
                                 kLayerBoundaryKey);
                }
            } else {
                bounds = infer_layer_boundaries(g);
            }
            clusters = split_layer_clusters(g, std::move(clusters), bounds, span);
        }
        for (const auto& cl : clusters) {
            std::vector<const OrtNode*> nodes;
            for (size_t i : cl) nodes.push_back(g.nodes[i].handle);
            OrtNodeFusionOptions opts{ORT_API_VERSION, true};
            check_ort(ep->api,
                      ep_api::EpGraphSupportInfo_AddNodesToFuse(ep->ep_api)(support, nodes.data(),
                                                                            nodes.size(), &opts),
                      "EpGraphSupportInfo_AddNodesToFuse");
        }
    });
}

OrtStatus* ep_compile(OrtEp* self, const OrtGraph** graphs, const OrtNode** fused_nodes,
                      size_t count, OrtNodeComputeInfo** infos, OrtNode** ep_context_nodes) {
    Ep* ep = reinterpret_cast<Ep*>(self);
    (void)ep_context_nodes;  // no EPContext serialisation (rust/src/ep.rs:957)
    for (size_t i = 0; i < count; ++i) infos[i] = nullptr;
    return guard(ep->api, "Compile", [&] {
        for (size_t i = 0; i < count; ++i) {
            const OrtApi* a = ep->api;
            GraphIR sub = read_graph(a, graphs[i]);
            // Kernel-context order = the fused node's input / output order.
            auto names = [&](auto count_fn, auto get_fn) {
                size_t n = 0;
                check_ort(a, count_fn(a)(fused_nodes[i], &n), "fused node io");
                std::vector<const OrtValueInfo*> vis(n);
                if (n) check_ort(a, get_fn(a)(fused_nodes[i], vis.data(), n), "fused node io");
                std::vector<std::string> out;
                for (auto* vi : vis) {
                    const char* nm = nullptr;
                    if (vi) check_ort(a, api::GetValueInfoName(a)(vi, &nm), "GetValueInfoName");
                    out.push_back(nm ? nm : "");
                }
                return out;
            };
            auto ins = names(api::Node_GetNumInputs, api::Node_GetInputs);
            auto outs = names(api::Node_GetNumOutputs, api::Node_GetOutputs);
            auto ci = new ComputeInfo();
            ci->base.ort_version_supported = ORT_API_VERSION;
            ci->base.CreateState = ci_create_state;
            ci->base.Compute = ci_compute;
            ci->base.ReleaseState = ci_release_state;
            ci->api = a;
            try {
                ci->plan = std::make_unique<Plan>(std::move(sub), ins, outs, ep->device);
            } catch (...) {
                delete ci;
                for (size_t j = 0; j < i; ++j) {
                    delete reinterpret_cast<ComputeInfo*>(infos[j]);
                    infos[j] = nullptr;
                }
                throw;
            }
            infos[i] = &ci->base;
        }
    });
}

void ep_release_infos(OrtEp*, OrtNodeComputeInfo** infos, size_t n) {
    for (size_t i = 0; i < n; ++i) delete reinterpret_cast<ComputeInfo*>(infos[i]);
}

// The HBM memory device registered on the EP device (f_supported_devices): ORT
// then places the fused nodes' inputs and outputs in HBM, copying host feeds in
// and host-bound outputs out through this EP's data transfer, and a KV cache bound
// to device buffers never crosses PCIe. ORTMI_EP_MEMORY=cpu reports CPU memory
// instead, the reference's answer on unified memory (rust/src/ep.rs:104-113): ORT
// then hands Compute host buffers, which the plan stages itself (host KV caches
// shared between past and present get only their new rows written back).
OrtStatus* ep_default_memory_device(const OrtEp* self, const OrtMemoryDevice** device) {
    if (device) *device = reinterpret_cast<const Ep*>(self)->memory_device;
    return nullptr;
}

// ---------------------------------------------------------------- factory --
Factory* F(const OrtEpFactory* p) { return reinterpret_cast<Factory*>(const_cast<OrtEpFactory*>(p)); }

const char* f_name(const OrtEpFactory* p) { return F(p)->name.c_str(); }
const char* f_vendor(const OrtEpFactory* p) { return F(p)->vendor.c_str(); }
uint32_t f_vendor_id(const OrtEpFactory*) { return kVendorIdAmd; }
const char* f_version(const OrtEpFactory* p) { return F(p)->version.c_str(); }
bool f_stream_aware(const OrtEpFactory*) { return false; }

OrtStatus* f_supported_devices(OrtEpFactory* p, const OrtHardwareDevice* const* devices,
                               size_t num_devices, OrtEpDevice** ep_devices, size_t max_ep_devices,
                               size_t* num_ep_devices) {
    Factory* f = F(p);
    return guard(f->api, "GetSupportedDevices", [&] {
        *num_ep_devices = 0;
        int hip_devices = 0;
        if (hipGetDeviceCount(&hip_devices) != hipSuccess) {
            (void)hipGetLastError();
            hip_devices = 0;
        }
        if (hip_devices <= 0 || max_ep_devices < 1) return;  // nothing to offer
        // First GPU hardware device (rust/src/factory.rs:116-164).
        const OrtHardwareDevice* gpu = nullptr;
        for (size_t i = 0; i < num_devices && !gpu; ++i)
            if (api::HardwareDevice_Type(f->api)(devices[i]) == OrtHardwareDeviceType_GPU)
                gpu = devices[i];
        if (!gpu) return;
        OrtEpDevice* d = nullptr;
        check_ort(f->api, ep_api::CreateEpDevice(f->ep_api)(p, gpu, nullptr, nullptr, &d),
                  "CreateEpDevice");
        // The device's memory: HBM of GPU 0 (AMD vendor id), device allocator.
        if (!f->hbm_info) {
            OrtStatus* st = api::CreateMemoryInfo_V2(f->api)(
                kHbmMemoryInfoName, OrtMemoryInfoDeviceType_GPU, kVendorIdAmd, 0,
                OrtDeviceMemoryType_DEFAULT, 256, OrtDeviceAllocator, &f->hbm_info);
            if (st) ep_api::ReleaseEpDevice(f->ep_api)(d);
            check_ort(f->api, st, "CreateMemoryInfo_V2");
        }
        OrtStatus* st = ep_api::EpDevice_AddAllocatorInfo(f->ep_api)(d, f->hbm_info);
        if (st) ep_api::ReleaseEpDevice(f->ep_api)(d);
        check_ort(f->api, st, "EpDevice_AddAllocatorInfo");
        ep_devices[0] = d;
        *num_ep_devices = 1;
    });
}

OrtStatus* f_create_ep(OrtEpFactory* p, const OrtHardwareDevice* const*,
                       const OrtKeyValuePairs* const*, size_t num_devices,
                       const OrtSessionOptions*, const OrtLogger*, OrtEp** out) {
    Factory* f = F(p);
    *out = nullptr;
    return guard(f->api, "CreateEp", [&] {
        if (num_devices != 1)
            fail("MI355XExecutionProvider expects exactly one device", ORT_INVALID_ARGUMENT);
        auto* ep = new Ep();
        std::memset(&ep->base, 0, sizeof(ep->base));
        ep->base.ort_version_supported = ORT_API_VERSION;
        ep->base.GetName = ep_get_name;
        ep->base.GetCapability = ep_get_capability;
        ep->base.Compile = ep_compile;
        ep->base.ReleaseNodeComputeInfos = ep_release_infos;
        ep->base.GetDefaultMemoryDevice = ep_default_memory_device;
        ep->factory = f;
        ep->api = f->api;
        ep->ep_api = f->ep_api;
        ep->name = f->name;
        ep->device = 0;
        const char* mem = std::getenv("ORTMI_EP_MEMORY");
        const bool cpu = mem && std::strcmp(mem, "cpu") == 0;
        if (!cpu && f->hbm_info)
            ep->memory_device = ep_api::MemoryInfo_GetMemoryDevice(f->ep_api)(f->hbm_info);
        *out = &ep->base;
    });
}

void f_release_ep(OrtEpFactory*, OrtEp* ep) { delete reinterpret_cast<Ep*>(ep); }

OrtStatus* f_create_allocator(OrtEpFactory* p, const OrtMemoryInfo* info, const OrtKeyValuePairs*,
                              OrtAllocator** out) {
    Factory* f = F(p);
    if (out) *out = nullptr;
    return guard(f->api, "CreateAllocator", [&] {
        if (!out) fail("null allocator output", ORT_INVALID_ARGUMENT);
        if (!info) return;
        const char* name = nullptr;
        check_ort(f->api, api::MemoryInfoGetName(f->api)(info, &name), "MemoryInfoGetName");
        if (!name || std::strcmp(name, kHbmMemoryInfoName) != 0) return;  // not this EP's memory
        int id = 0;
        check_ort(f->api, api::MemoryInfoGetId(f->api)(info, &id), "MemoryInfoGetId");
        int count = 0;
        if (hipGetDeviceCount(&count) != hipSuccess) {
            (void)hipGetLastError();
            count = 0;
        }
        if (id < 0 || id >= count)
            fail("memory info names GPU " + std::to_string(id) + ", but " +
                     std::to_string(count) + " are visible",
                 ORT_INVALID_ARGUMENT);
        auto* a = new DeviceAllocator();
        std::memset(&a->base, 0, sizeof(a->base));
        // GetStats stays null: ORT's allocator wrapper calls it only when set, and
        // this allocator keeps no statistics of its own.
        a->base.version = ORT_API_VERSION;
        a->base.Alloc = alloc_fn;
        a->base.Free = free_fn;
        a->base.Info = info_fn;
        a->base.Reserve = reserve_fn;
        a->base.AllocOnStream = alloc_on_stream_fn;
        a->info = info;
        a->device = id;
        *out = &a->base;
    });
}
void f_release_allocator(OrtEpFactory*, OrtAllocator* a) {
    delete reinterpret_cast<DeviceAllocator*>(a);
}
OrtStatus* f_create_data_transfer(OrtEpFactory* p, OrtDataTransferImpl** out) {
    Factory* f = F(p);
    return guard(f->api, "CreateDataTransfer", [&] {
        auto* t = new DataTransfer();
        t->base.ort_version_supported = ORT_API_VERSION;
        t->base.Release = dt_release;
        t->base.CanCopy = dt_can_copy;
        t->base.CopyTensors = dt_copy;
        t->api = f->api;
        t->ep_api = f->ep_api;
        *out = &t->base;
    });
}
OrtStatus* f_create_stream(OrtEpFactory*, const OrtMemoryDevice*, const OrtKeyValuePairs*,
                           OrtSyncStreamImpl** out) {
    *out = nullptr;  // not stream aware
    return nullptr;
}

}  // namespace
}  // namespace ortmi_ep

using namespace ortmi_ep;

// Entry point resolved by ORT through dlsym (rust/src/lib.rs:90-155).
ORTMI_EXPORT OrtStatus* CreateEpFactories(const char* registration_name,
                                          const OrtApiBase* ort_api_base,
                                          const OrtLogger* default_logger,
                                          OrtEpFactory** factories, size_t max_factories,
                                          size_t* num_factories) {
    (void)default_logger;
    if (num_factories) *num_factories = 0;
    // Without an API base no status can be created: report zero factories.
    if (!ort_api_base || !ort_api_base->GetApi) return nullptr;
    const OrtApi* a = ort_api_base->GetApi(ORT_API_VERSION);
    if (!a) {
        const OrtApi* legacy = ort_api_base->GetApi(1);
        if (!legacy) return nullptr;
        return api::CreateStatus(legacy)(
            ORT_INVALID_ARGUMENT, "MI355XExecutionProvider requires ONNX Runtime with ORT_API_VERSION >= 29");
    }
    return guard(a, "CreateEpFactories", [&] {
        if (!factories || !num_factories) fail("null output arguments", ORT_INVALID_ARGUMENT);
        *num_factories = 0;
        if (max_factories < 1)
            fail("MI355XExecutionProvider needs room for one OrtEpFactory", ORT_INVALID_ARGUMENT);
        auto* f = new Factory();
        std::memset(&f->base, 0, sizeof(f->base));
        f->api = a;
        f->ep_api = api::GetEpApi(a)();
        f->name = (registration_name && *registration_name) ? registration_name : kDefaultName;
        f->vendor = "AMD";
        f->version = kVersion;
        OrtEpFactory& b = f->base;
        b.ort_version_supported = ORT_API_VERSION;
        b.GetName = f_name;
        b.GetVendor = f_vendor;
        b.GetVendorId = f_vendor_id;
        b.GetVersion = f_version;
        b.GetSupportedDevices = f_supported_devices;
        b.CreateEp = f_create_ep;
        b.ReleaseEp = f_release_ep;
        b.CreateAllocator = f_create_allocator;
        b.ReleaseAllocator = f_release_allocator;
        b.CreateDataTransfer = f_create_data_transfer;
        b.IsStreamAware = f_stream_aware;
        b.CreateSyncStreamForDevice = f_create_stream;
        factories[0] = &f->base;
        *num_factories = 1;
    });
}

// rust/src/lib.rs:161-167
ORTMI_EXPORT OrtStatus* ReleaseEpFactory(OrtEpFactory* factory) {
    delete reinterpret_cast<Factory*>(factory);
    return nullptr;
}
