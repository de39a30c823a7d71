/*
 * ort_plugin_ep_abi.h - the subset of ONNX Runtime's plugin execution-provider C ABI
 * (onnxruntime_c_api.h / onnxruntime_ep_c_api.h, ORT_API_VERSION 29) that the MI355X
 * EP implements and calls.
 *
 * The reference EP binds the same ABI through bindgen over ORT's headers
 * (rust/wrapper_ort.h, rust/build.rs:63-74) and exports exactly two symbols,
 * CreateEpFactories and ReleaseEpFactory (rust/src/lib.rs:90-167); it reaches
 * every other ORT function through the OrtApi / OrtEpApi tables handed to
 * CreateEpFactories, without linking libonnxruntime (rust/build.rs:89-90). This
 * header restates the struct layouts and the function-table slots that EP needs.
 *
 * ORT's headers are not part of this repository; the layouts below follow their
 * published declarations. Every function-table slot index used anywhere in this
 * project is listed once, in ORTMI_ORT_API_SLOTS / ORTMI_ORT_EP_API_SLOTS below,
 * so that a check against a real onnxruntime_c_api.h touches a single table.
 */
#ifndef ORT_PLUGIN_EP_ABI_H
#define ORT_PLUGIN_EP_ABI_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORT_API_VERSION 29

/* ------------------------------------------------------------ opaque types */
typedef struct OrtStatus OrtStatus;
typedef struct OrtLogger OrtLogger;
typedef struct OrtHardwareDevice OrtHardwareDevice;
typedef struct OrtEpDevice OrtEpDevice;
typedef struct OrtKeyValuePairs OrtKeyValuePairs;
typedef struct OrtSessionOptions OrtSessionOptions;
typedef struct OrtMemoryInfo OrtMemoryInfo;
typedef struct OrtMemoryDevice OrtMemoryDevice;
typedef struct OrtGraph OrtGraph;
typedef struct OrtNode OrtNode;
typedef struct OrtValueInfo OrtValueInfo;
typedef struct OrtValue OrtValue;
typedef struct OrtOpAttr OrtOpAttr;
typedef struct OrtKernelContext OrtKernelContext;
typedef struct OrtTypeInfo OrtTypeInfo;
typedef struct OrtTensorTypeAndShapeInfo OrtTensorTypeAndShapeInfo;
typedef struct OrtEpGraphSupportInfo OrtEpGraphSupportInfo;
typedef struct OrtNodeComputeContext OrtNodeComputeContext;
typedef struct OrtModelMetadata OrtModelMetadata;
typedef struct OrtSyncStreamImpl OrtSyncStreamImpl;
typedef struct OrtApi OrtApi;
typedef struct OrtEpApi OrtEpApi;

/* ------------------------------------------------------------------- enums */
typedef enum OrtErrorCode {
    ORT_OK = 0,
    ORT_FAIL = 1,
    ORT_INVALID_ARGUMENT = 2,
    ORT_NO_SUCHFILE = 3,
    ORT_NO_MODEL = 4,
    ORT_ENGINE_ERROR = 5,
    ORT_RUNTIME_EXCEPTION = 6,
    ORT_INVALID_PROTOBUF = 7,
    ORT_MODEL_LOADED = 8,
    ORT_NOT_IMPLEMENTED = 9,
    ORT_INVALID_GRAPH = 10,
    ORT_EP_FAIL = 11,
    ORT_MODEL_LOAD_CANCELED = 12,
    ORT_MODEL_REQUIRES_COMPILATION = 13,
    ORT_NOT_FOUND = 14,
} OrtErrorCode;

typedef enum ONNXTensorElementDataType {
    ONNX_TENSOR_ELEMENT_DATA_TYPE_UNDEFINED = 0,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT = 1,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_UINT8 = 2,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_INT8 = 3,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_UINT16 = 4,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_INT16 = 5,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_INT32 = 6,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_INT64 = 7,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_STRING = 8,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_BOOL = 9,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_FLOAT16 = 10,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_DOUBLE = 11,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_UINT32 = 12,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_UINT64 = 13,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_COMPLEX64 = 14,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_COMPLEX128 = 15,
    ONNX_TENSOR_ELEMENT_DATA_TYPE_BFLOAT16 = 16,
} ONNXTensorElementDataType;

typedef enum ONNXType {
    ONNX_TYPE_UNKNOWN = 0,
    ONNX_TYPE_TENSOR = 1,
    ONNX_TYPE_SEQUENCE = 2,
    ONNX_TYPE_MAP = 3,
    ONNX_TYPE_OPAQUE = 4,
    ONNX_TYPE_SPARSETENSOR = 5,
    ONNX_TYPE_OPTIONAL = 6,
} ONNXType;

typedef enum OrtOpAttrType {
    ORT_OP_ATTR_UNDEFINED = 0,
    ORT_OP_ATTR_INT = 1,
    ORT_OP_ATTR_INTS = 2,
    ORT_OP_ATTR_FLOAT = 3,
    ORT_OP_ATTR_FLOATS = 4,
    ORT_OP_ATTR_STRING = 5,
    ORT_OP_ATTR_STRINGS = 6,
    ORT_OP_ATTR_GRAPH = 7,
    ORT_OP_ATTR_TENSOR = 8,
} OrtOpAttrType;

typedef enum OrtHardwareDeviceType {
    OrtHardwareDeviceType_CPU = 0,
    OrtHardwareDeviceType_GPU = 1,
    OrtHardwareDeviceType_NPU = 2,
} OrtHardwareDeviceType;

typedef enum OrtAllocatorType {
    OrtInvalidAllocator = -1,
    OrtDeviceAllocator = 0,
    OrtArenaAllocator = 1,
} OrtAllocatorType;

typedef enum OrtMemType {
    OrtMemTypeCPUInput = -2,
    OrtMemTypeCPUOutput = -1,
    OrtMemTypeDefault = 0,
} OrtMemType;

typedef enum OrtDeviceMemoryType {
    OrtDeviceMemoryType_DEFAULT = 0,
    OrtDeviceMemoryType_HOST_ACCESSIBLE = 5,
} OrtDeviceMemoryType;

typedef enum OrtMemoryInfoDeviceType {
    OrtMemoryInfoDeviceType_CPU = 0,
    OrtMemoryInfoDeviceType_GPU = 1,
    OrtMemoryInfoDeviceType_FPGA = 2,
    OrtMemoryInfoDeviceType_NPU = 3,
} OrtMemoryInfoDeviceType;

/* ----------------------------------------------------------- plain structs */
typedef struct OrtApiBase {
    const OrtApi* (*GetApi)(uint32_t version);
    const char* (*GetVersionString)(void);
} OrtApiBase;

/* OrtAllocator: version + function pointers (onnxruntime_c_api.h). */
typedef struct OrtAllocator {
    uint32_t version;
    void* (*Alloc)(struct OrtAllocator* this_, size_t size);
    void (*Free)(struct OrtAllocator* this_, void* p);
    const OrtMemoryInfo* (*Info)(const struct OrtAllocator* this_);
    void* (*Reserve)(struct OrtAllocator* this_, size_t size);
    OrtStatus* (*GetStats)(const struct OrtAllocator* this_, OrtKeyValuePairs** out);
    void* (*AllocOnStream)(struct OrtAllocator* this_, size_t size, OrtSyncStreamImpl* stream);
} OrtAllocator;

/* OrtDataTransferImpl: host <-> device copies for the EP's memory device. */
typedef struct OrtDataTransferImpl {
    uint32_t ort_version_supported;
    void (*Release)(struct OrtDataTransferImpl* this_ptr);
    bool (*CanCopy)(const struct OrtDataTransferImpl* this_ptr, const OrtMemoryDevice* src,
                    const OrtMemoryDevice* dst);
    OrtStatus* (*CopyTensors)(struct OrtDataTransferImpl* this_ptr, const OrtValue** src_tensors,
                              OrtValue** dst_tensors, OrtSyncStreamImpl** streams,
                              size_t num_tensors);
} OrtDataTransferImpl;

typedef struct OrtNodeFusionOptions {
    uint32_t ort_version_supported;
    bool drop_constant_initializers;
} OrtNodeFusionOptions;

typedef struct OrtNodeComputeInfo {
    uint32_t ort_version_supported;
    OrtStatus* (*CreateState)(struct OrtNodeComputeInfo* this_ptr,
                              OrtNodeComputeContext* compute_context, void** compute_state);
    OrtStatus* (*Compute)(struct OrtNodeComputeInfo* this_ptr, void* compute_state,
                          OrtKernelContext* kernel_context);
    void (*ReleaseState)(struct OrtNodeComputeInfo* this_ptr, void* compute_state);
} OrtNodeComputeInfo;

typedef struct OrtEp {
    uint32_t ort_version_supported;
    const char* (*GetName)(const struct OrtEp* this_ptr);
    OrtStatus* (*GetCapability)(struct OrtEp* this_ptr, const OrtGraph* graph,
                                OrtEpGraphSupportInfo* graph_support_info);
    OrtStatus* (*Compile)(struct OrtEp* this_ptr, const OrtGraph** graphs,
                          const OrtNode** fused_nodes, size_t count,
                          OrtNodeComputeInfo** node_compute_infos, OrtNode** ep_context_nodes);
    void (*ReleaseNodeComputeInfos)(struct OrtEp* this_ptr, OrtNodeComputeInfo** node_compute_infos,
                                    size_t num_node_compute_infos);
    OrtStatus* (*GetPreferredDataLayout)(struct OrtEp* this_ptr, int* preferred_data_layout);
    OrtStatus* (*ShouldConvertDataLayoutForOp)(struct OrtEp* this_ptr, const char* domain,
                                               const char* op_type, int target_data_layout,
                                               int* should_convert);
    OrtStatus* (*SetDynamicOptions)(struct OrtEp* this_ptr, const char* const* option_keys,
                                    const char* const* option_values, size_t num_options);
    OrtStatus* (*OnRunStart)(struct OrtEp* this_ptr, const void* run_options);
    OrtStatus* (*OnRunEnd)(struct OrtEp* this_ptr, const void* run_options, bool sync_stream);
    OrtStatus* (*CreateAllocator)(struct OrtEp* this_ptr, const OrtMemoryInfo* memory_info,
                                  OrtAllocator** allocator);
    OrtStatus* (*CreateSyncStreamForDevice)(struct OrtEp* this_ptr,
                                            const OrtMemoryDevice* memory_device,
                                            OrtSyncStreamImpl** stream);
    const char* (*GetCompiledModelCompatibilityInfo)(struct OrtEp* this_ptr, const OrtGraph* graph);
    /* Memory device the EP's inputs and outputs should live on; *device = NULL
     * means CPU memory (rust/src/ep.rs:104-113 binds this exact type). */
    OrtStatus* (*GetDefaultMemoryDevice)(const struct OrtEp* this_ptr,
                                         const OrtMemoryDevice** device);
} OrtEp;

typedef struct OrtEpFactory {
    uint32_t ort_version_supported;
    const char* (*GetName)(const struct OrtEpFactory* this_ptr);
    const char* (*GetVendor)(const struct OrtEpFactory* this_ptr);
    OrtStatus* (*GetSupportedDevices)(struct OrtEpFactory* this_ptr,
                                      const OrtHardwareDevice* const* devices, size_t num_devices,
                                      OrtEpDevice** ep_devices, size_t max_ep_devices,
                                      size_t* num_ep_devices);
    OrtStatus* (*CreateEp)(struct OrtEpFactory* this_ptr, const OrtHardwareDevice* const* devices,
                           const OrtKeyValuePairs* const* ep_metadata_pairs, size_t num_devices,
                           const OrtSessionOptions* session_options, const OrtLogger* logger,
                           OrtEp** ep);
    void (*ReleaseEp)(struct OrtEpFactory* this_ptr, OrtEp* ep);
    uint32_t (*GetVendorId)(const struct OrtEpFactory* this_ptr);
    const char* (*GetVersion)(const struct OrtEpFactory* this_ptr);
    OrtStatus* (*ValidateCompiledModelCompatibilityInfo)(struct OrtEpFactory* this_ptr,
                                                         const OrtHardwareDevice* const* devices,
                                                         size_t num_devices,
                                                         const char* compatibility_info,
                                                         int* model_compatibility);
    OrtStatus* (*CreateAllocator)(struct OrtEpFactory* this_ptr, const OrtMemoryInfo* memory_info,
                                  const OrtKeyValuePairs* allocator_options,
                                  OrtAllocator** allocator);
    void (*ReleaseAllocator)(struct OrtEpFactory* this_ptr, OrtAllocator* allocator);
    OrtStatus* (*CreateDataTransfer)(struct OrtEpFactory* this_ptr,
                                     OrtDataTransferImpl** data_transfer);
    bool (*IsStreamAware)(const struct OrtEpFactory* this_ptr);
    OrtStatus* (*CreateSyncStreamForDevice)(struct OrtEpFactory* this_ptr,
                                            const OrtMemoryDevice* memory_device,
                                            const OrtKeyValuePairs* stream_options,
                                            OrtSyncStreamImpl** stream);
} OrtEpFactory;

/* ------------------------------------------------------ function-table slots
 * X(slot, name, return type, (parameter list)). OrtApi and OrtEpApi are arrays
 * of function pointers in ORT's declaration order; only the slots below are
 * called (by the EP) or provided (by the in-repo harness host). */
#define ORTMI_ORT_API_SLOTS(X)                                                                    \
    X(0, CreateStatus, OrtStatus*, (OrtErrorCode code, const char* msg))                         \
    X(1, GetErrorCode, OrtErrorCode, (const OrtStatus* status))                                  \
    X(2, GetErrorMessage, const char*, (const OrtStatus* status))                                \
    X(51, GetTensorMutableData, OrtStatus*, (OrtValue* value, void** out))                       \
    X(55, CastTypeInfoToTensorInfo, OrtStatus*,                                                  \
      (const OrtTypeInfo* type_info, const OrtTensorTypeAndShapeInfo** out))                     \
    X(56, GetOnnxTypeFromTypeInfo, OrtStatus*, (const OrtTypeInfo* type_info, ONNXType* out))    \
    X(60, GetTensorElementType, OrtStatus*,                                                      \
      (const OrtTensorTypeAndShapeInfo* info, ONNXTensorElementDataType* out))                   \
    X(61, GetDimensionsCount, OrtStatus*, (const OrtTensorTypeAndShapeInfo* info, size_t* out))  \
    X(62, GetDimensions, OrtStatus*,                                                             \
      (const OrtTensorTypeAndShapeInfo* info, int64_t* dims, size_t dims_len))                   \
    X(64, GetTensorShapeElementCount, OrtStatus*,                                                \
      (const OrtTensorTypeAndShapeInfo* info, size_t* out))                                      \
    X(65, GetTensorTypeAndShape, OrtStatus*, (const OrtValue* value,                             \
                                              OrtTensorTypeAndShapeInfo** out))                  \
    X(68, CreateMemoryInfo, OrtStatus*,                                                          \
      (const char* name, OrtAllocatorType type, int id, OrtMemType mem_type,                    \
       OrtMemoryInfo** out))                                                                    \
    X(71, MemoryInfoGetName, OrtStatus*, (const OrtMemoryInfo* info, const char** out))          \
    X(72, MemoryInfoGetId, OrtStatus*, (const OrtMemoryInfo* info, int* out))                    \
    X(78, GetAllocatorWithDefaultOptions, OrtStatus*, (OrtAllocator * *out))                     \
    X(88, KernelContext_GetInputCount, OrtStatus*, (const OrtKernelContext* ctx, size_t* out))   \
    X(89, KernelContext_GetOutputCount, OrtStatus*, (const OrtKernelContext* ctx, size_t* out))  \
    X(90, KernelContext_GetInput, OrtStatus*,                                                    \
      (const OrtKernelContext* ctx, size_t index, const OrtValue** out))                         \
    X(91, KernelContext_GetOutput, OrtStatus*,                                                   \
      (OrtKernelContext * ctx, size_t index, const int64_t* dims, size_t dim_count,              \
       OrtValue** out))                                                                          \
    X(93, ReleaseStatus, void, (OrtStatus * status))                                             \
    X(94, ReleaseMemoryInfo, void, (OrtMemoryInfo * info))                                       \
    X(99, ReleaseTensorTypeAndShapeInfo, void, (OrtTensorTypeAndShapeInfo * info))               \
    X(116, ModelMetadataLookupCustomMetadataMap, OrtStatus*,                                     \
      (const OrtModelMetadata* model_metadata, OrtAllocator* allocator, const char* key,         \
       char** value))                                                                            \
    X(118, ReleaseModelMetadata, void, (OrtModelMetadata * model_metadata))                      \
    X(285, GetEpApi, const OrtEpApi*, (void))                                                    \
    X(286, HardwareDevice_Type, OrtHardwareDeviceType, (const OrtHardwareDevice* device))        \
    X(301, GetTensorData, OrtStatus*, (const OrtValue* value, const void** out))                 \
    X(317, CreateMemoryInfo_V2, OrtStatus*,                                                      \
      (const char* name, OrtMemoryInfoDeviceType device_type, uint32_t vendor_id,                \
       int32_t device_id, OrtDeviceMemoryType mem_type, size_t alignment,                        \
       OrtAllocatorType allocator_type, OrtMemoryInfo** out))                                   \
    X(310, GetValueInfoName, OrtStatus*, (const OrtValueInfo* value_info, const char** name))    \
    X(311, GetValueInfoTypeInfo, OrtStatus*,                                                     \
      (const OrtValueInfo* value_info, const OrtTypeInfo** type_info))                           \
    X(320, ValueInfo_GetValueProducer, OrtStatus*,                                               \
      (const OrtValueInfo* value_info, const OrtNode** producer, size_t* output_index))          \
    X(324, ValueInfo_GetInitializerValue, OrtStatus*,                                            \
      (const OrtValueInfo* value_info, const OrtValue** value))                                  \
    X(327, ValueInfo_IsConstantInitializer, OrtStatus*,                                          \
      (const OrtValueInfo* value_info, bool* is_constant))                                       \
    X(335, Graph_GetNumInputs, OrtStatus*, (const OrtGraph* graph, size_t* out))                 \
    X(336, Graph_GetInputs, OrtStatus*,                                                          \
      (const OrtGraph* graph, const OrtValueInfo** inputs, size_t num))                          \
    X(337, Graph_GetNumOutputs, OrtStatus*, (const OrtGraph* graph, size_t* out))                \
    X(338, Graph_GetOutputs, OrtStatus*,                                                         \
      (const OrtGraph* graph, const OrtValueInfo** outputs, size_t num))                         \
    X(339, Graph_GetNumInitializers, OrtStatus*, (const OrtGraph* graph, size_t* out))           \
    X(340, Graph_GetInitializers, OrtStatus*,                                                    \
      (const OrtGraph* graph, const OrtValueInfo** initializers, size_t num))                    \
    X(341, Graph_GetNumNodes, OrtStatus*, (const OrtGraph* graph, size_t* out))                  \
    X(342, Graph_GetNodes, OrtStatus*, (const OrtGraph* graph, const OrtNode** nodes,            \
                                        size_t num))                                             \
    X(343, Graph_GetParentNode, OrtStatus*, (const OrtGraph* graph, const OrtNode** node))       \
    X(345, Graph_GetModelMetadata, OrtStatus*,                                                   \
      (const OrtGraph* graph, OrtModelMetadata** out))                                           \
    X(348, Node_GetId, OrtStatus*, (const OrtNode* node, size_t* id))                            \
    X(349, Node_GetName, OrtStatus*, (const OrtNode* node, const char** name))                   \
    X(350, Node_GetOperatorType, OrtStatus*, (const OrtNode* node, const char** op_type))        \
    X(351, Node_GetDomain, OrtStatus*, (const OrtNode* node, const char** domain))               \
    X(352, Node_GetSinceVersion, OrtStatus*, (const OrtNode* node, int* since_version))          \
    X(353, Node_GetNumInputs, OrtStatus*, (const OrtNode* node, size_t* out))                    \
    X(354, Node_GetInputs, OrtStatus*,                                                           \
      (const OrtNode* node, const OrtValueInfo** inputs, size_t num))                            \
    X(355, Node_GetNumOutputs, OrtStatus*, (const OrtNode* node, size_t* out))                   \
    X(356, Node_GetOutputs, OrtStatus*,                                                          \
      (const OrtNode* node, const OrtValueInfo** outputs, size_t num))                           \
    X(361, Node_GetNumAttributes, OrtStatus*, (const OrtNode* node, size_t* out))                \
    X(362, Node_GetAttributes, OrtStatus*,                                                       \
      (const OrtNode* node, const OrtOpAttr** attributes, size_t num))                           \
    X(363, Node_GetAttributeByName, OrtStatus*,                                                  \
      (const OrtNode* node, const char* name, const OrtOpAttr** attribute))                      \
    X(365, OpAttr_GetType, OrtStatus*, (const OrtOpAttr* attribute, OrtOpAttrType* type))        \
    X(366, OpAttr_GetName, OrtStatus*, (const OrtOpAttr* attribute, const char** name))          \
    X(367, ReadOpAttr, OrtStatus*,                                                               \
      (const OrtOpAttr* attribute, OrtOpAttrType type, void* data, size_t len, size_t* out))

#define ORTMI_ORT_EP_API_SLOTS(X)                                                                 \
    X(0, CreateEpDevice, OrtStatus*,                                                             \
      (OrtEpFactory * factory, const OrtHardwareDevice* hardware_device,                         \
       const OrtKeyValuePairs* ep_metadata, const OrtKeyValuePairs* ep_options,                  \
       OrtEpDevice** ep_device))                                                                 \
    X(1, ReleaseEpDevice, void, (OrtEpDevice * device))                                          \
    X(2, EpGraphSupportInfo_AddNodesToFuse, OrtStatus*,                                          \
      (OrtEpGraphSupportInfo * info, const OrtNode* const* nodes, size_t num_nodes,              \
       const OrtNodeFusionOptions* options))                                                     \
    X(3, EpGraphSupportInfo_AddSingleNode, OrtStatus*,                                           \
      (OrtEpGraphSupportInfo * info, const OrtNode* node))                                       \
    X(4, NodeComputeContext_NodeName, const char*, (const OrtNodeComputeContext* context))       \
    X(5, EpDevice_AddAllocatorInfo, OrtStatus*,                                                  \
      (OrtEpDevice * ep_device, const OrtMemoryInfo* allocator_memory_info))                     \
    X(6, MemoryInfo_GetMemoryDevice, const OrtMemoryDevice*, (const OrtMemoryInfo* memory_info)) \
    X(9, MemoryDevice_GetDeviceType, OrtMemoryInfoDeviceType, (const OrtMemoryDevice* device))   \
    X(11, MemoryDevice_GetVendorId, uint32_t, (const OrtMemoryDevice* device))                   \
    X(12, MemoryDevice_GetDeviceId, uint32_t, (const OrtMemoryDevice* device))

/* Upper bounds of the slot numbers above (sizes of a table that holds them). */
#define ORTMI_ORT_API_TABLE_SIZE 400
#define ORTMI_ORT_EP_API_TABLE_SIZE 64

/* Plugin entry points (rust/src/lib.rs:90-167). */
typedef OrtStatus* (*CreateEpFactoriesFn)(const char* registration_name,
                                          const OrtApiBase* ort_api_base,
                                          const OrtLogger* default_logger,
                                          OrtEpFactory** factories, size_t max_factories,
                                          size_t* num_factories);
typedef OrtStatus* (*ReleaseEpFactoryFn)(OrtEpFactory* factory);

#ifdef __cplusplus
}

/* C++ accessors: ort::api::Name(api)(args...) calls slot `Name` of the table. */
namespace ort_abi {
#define ORTMI_DECLARE_ACCESSOR(slot, name, ret, params)                                \
    typedef ret(*name##_fn) params;                                                    \
    inline name##_fn name(const void* table) {                                         \
        return reinterpret_cast<name##_fn>(reinterpret_cast<void* const*>(table)[slot]); \
    }                                                                                  \
    enum : int { name##_slot = slot };
namespace api {
ORTMI_ORT_API_SLOTS(ORTMI_DECLARE_ACCESSOR)
}
namespace ep_api {
ORTMI_ORT_EP_API_SLOTS(ORTMI_DECLARE_ACCESSOR)
}
#undef ORTMI_DECLARE_ACCESSOR
}  // namespace ort_abi
#endif

#endif
