// A mock ONNX Runtime host for the MI355X plugin EP — TEST INFRASTRUCTURE.
//
// It plays ORT's side of the plugin-EP ABI the way the reference's Rust mock host does
// (rust/tests/mock_ort/mod.rs:1-60, driven through dlopen in rust/tests/cdylib_load.rs:1-50):
// an OrtApiBase whose OrtApi / OrtEpApi implement only the calls an EP may make, over an
// in-memory graph, so the library is loaded by `dlopen` and driven through CreateEpFactories ->
// GetSupportedDevices -> CreateEp -> GetCapability -> Compile -> Compute exactly as ORT would.
// Every slot the mock does not implement is NULL, so an EP that calls outside the contract
// crashes the test instead of passing it.  Contract checks recorded for the tests:
//   * every OrtStatus the mock creates is released exactly once (live count returns to 0);
//   * out-parameters are written before any failure (Compile's infos are NULL or valid);
//   * the EP only fuses nodes of the graph it was handed.
// The API version the mock offers is selectable, to exercise ABI negotiation.
//
// Exposed to Python (ctypes) through the mock_* functions at the end of this file.
#include <dlfcn.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <set>
#include <string>
#include <vector>

#include "onnxruntime_c_api.h"

// ---- the opaque ORT objects, as this host defines them ----------------------------------------

struct OrtStatus {
    OrtErrorCode code;
    std::string msg;
};
struct OrtTensorTypeAndShapeInfo {
    int32_t elem = 0;
    std::vector<int64_t> dims;
};
struct OrtTypeInfo {
    OrtTensorTypeAndShapeInfo tensor;
};
struct OrtValueInfo {
    std::string name;
    OrtTypeInfo type;
    bool constant = false;
    std::vector<uint8_t> init;       // initializer bytes when constant
};
struct OrtMemoryDevice {
    OrtMemoryInfoDeviceType type;
    OrtDeviceMemoryType mem;
    uint32_t vendor;
    int32_t id;
};
struct OrtMemoryInfo {
    std::string name;
    OrtMemoryDevice dev;
    size_t alignment;
    OrtAllocatorType alloc_type;
};
static const OrtMemoryDevice kHostDevice{OrtMemoryInfoDeviceType_CPU, OrtDeviceMemoryType_DEFAULT, 0, 0};
struct OrtValue {
    int32_t elem = 0;
    std::vector<int64_t> dims;
    const void* data = nullptr;      // borrowed (inputs, initializers) or owned (outputs)
    std::vector<uint8_t> owned;
    size_t bytes = 0;
    const OrtMemoryDevice* md = &kHostDevice;   // where `data` lives
};
struct OrtOpAttr {
    std::string name;
    OrtOpAttrType type = ORT_OP_ATTR_INT;
    int64_t value = 0;
    float fvalue = 0.f;
    std::string svalue;
};
struct OrtNode {
    std::string op_type, domain, name;
    std::vector<OrtValueInfo*> inputs;   // nullptr for an absent optional input
    std::vector<OrtValueInfo*> outputs;
    std::vector<OrtOpAttr> attrs;
};
struct OrtGraph {
    std::vector<OrtNode*> nodes;
    OrtNode* parent = nullptr;
};
struct OrtKeyValuePairs {
    std::map<std::string, std::string> kv;
    std::vector<const char*> keys, values;
};
struct OrtHardwareDevice {
    OrtHardwareDeviceType type;
    uint32_t vendor_id, device_id;
};
struct OrtEpDevice {
    OrtEpFactory* factory;
    const OrtHardwareDevice* hw;
    OrtKeyValuePairs meta;
    std::vector<const OrtMemoryInfo*> alloc_infos;   // EpDevice_AddAllocatorInfo (borrowed, as ORT)
};
struct OrtEpGraphSupportInfo {
    const OrtGraph* graph;
    std::vector<std::vector<const OrtNode*>> groups;
    std::vector<bool> drop;
};
struct OrtSessionOptions {
    std::map<std::string, std::string> config;
};
struct OrtKernelContext {
    std::vector<OrtValue*> inputs;
    std::vector<std::unique_ptr<OrtValue>> outputs;
    std::vector<int32_t> out_elem;
    void* stream = nullptr;         // the EP stream's native handle (stream-aware EPs)
};
// ORT's framework stream wrapping an EP's OrtSyncStreamImpl.
struct OrtSyncStream {
    OrtSyncStreamImpl* impl = nullptr;
};
struct OrtLogger {};
struct OrtNodeComputeContext {};

namespace {

std::string g_err;
long g_live_status = 0;
long g_created_status = 0;
std::set<const OrtStatus*> g_status_set;
bool g_bad_release = false;

void set_err(const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
}

OrtStatus* mk_status(OrtErrorCode code, const std::string& msg) {
    OrtStatus* s = new OrtStatus{code, msg};
    ++g_live_status;
    ++g_created_status;
    g_status_set.insert(s);
    return s;
}

// ---- OrtApi implementation -----------------------------------------------------------------

#define NX noexcept

OrtStatus* ORT_API_CALL m_CreateStatus(OrtErrorCode code, const char* msg) NX {
    return mk_status(code, msg ? msg : "");
}
OrtErrorCode ORT_API_CALL m_GetErrorCode(const OrtStatus* s) NX { return s->code; }
const char* ORT_API_CALL m_GetErrorMessage(const OrtStatus* s) NX { return s->msg.c_str(); }
void ORT_API_CALL m_ReleaseStatus(OrtStatus* s) NX {
    if (!s) return;
    if (!g_status_set.count(s)) {
        g_bad_release = true;   // double release or a foreign pointer
        return;
    }
    g_status_set.erase(s);
    --g_live_status;
    delete s;
}

OrtStatus* ORT_API_CALL m_Graph_GetNumNodes(const OrtGraph* g, size_t* n) NX {
    *n = g->nodes.size();
    return nullptr;
}
OrtStatus* ORT_API_CALL m_Graph_GetNodes(const OrtGraph* g, const OrtNode** out, size_t n) NX {
    if (n < g->nodes.size()) return mk_status(ORT_INVALID_ARGUMENT, "node array too small");
    for (size_t i = 0; i < g->nodes.size(); ++i) out[i] = g->nodes[i];
    return nullptr;
}
OrtStatus* ORT_API_CALL m_Graph_GetParentNode(const OrtGraph* g, const OrtNode** out) NX {
    *out = g->parent;
    return nullptr;
}
OrtStatus* ORT_API_CALL m_Node_GetName(const OrtNode* n, const char** out) NX {
    *out = n->name.c_str();
    return nullptr;
}
OrtStatus* ORT_API_CALL m_Node_GetOperatorType(const OrtNode* n, const char** out) NX {
    *out = n->op_type.c_str();
    return nullptr;
}
OrtStatus* ORT_API_CALL m_Node_GetDomain(const OrtNode* n, const char** out) NX {
    *out = n->domain.c_str();
    return nullptr;
}
OrtStatus* ORT_API_CALL m_Node_GetNumInputs(const OrtNode* n, size_t* out) NX {
    *out = n->inputs.size();
    return nullptr;
}
OrtStatus* ORT_API_CALL m_Node_GetInputs(const OrtNode* n, const OrtValueInfo** out, size_t k) NX {
    if (k < n->inputs.size()) return mk_status(ORT_INVALID_ARGUMENT, "input array too small");
    for (size_t i = 0; i < n->inputs.size(); ++i) out[i] = n->inputs[i];
    return nullptr;
}
OrtStatus* ORT_API_CALL m_Node_GetNumOutputs(const OrtNode* n, size_t* out) NX {
    *out = n->outputs.size();
    return nullptr;
}
OrtStatus* ORT_API_CALL m_Node_GetOutputs(const OrtNode* n, const OrtValueInfo** out, size_t k) NX {
    if (k < n->outputs.size()) return mk_status(ORT_INVALID_ARGUMENT, "output array too small");
    for (size_t i = 0; i < n->outputs.size(); ++i) out[i] = n->outputs[i];
    return nullptr;
}
OrtStatus* ORT_API_CALL m_Node_GetAttributeByName(const OrtNode* n, const char* name,
                                                  const OrtOpAttr** out) NX {
    *out = nullptr;
    for (const OrtOpAttr& a : n->attrs)
        if (a.name == name) {
            *out = &a;
            return nullptr;
        }
    static const char* known[] = {"K", "N", "bits", "block_size", "accuracy_level", "weight_prepacked"};
    for (const char* k : known)
        if (!std::strcmp(k, name)) return nullptr;     // unset optional attribute
    return mk_status(ORT_NOT_FOUND, std::string("no attribute ") + name);
}
OrtStatus* ORT_API_CALL m_ReadOpAttr(const OrtOpAttr* a, OrtOpAttrType type, void* data, size_t len,
                                     size_t* out) NX {
    // as ORT: the requested type must be the attribute's; `out` is the byte count needed (on
    // failure) or written (on success); strings are written without a terminator
    if (type != a->type) return mk_status(ORT_INVALID_ARGUMENT, "attribute type mismatch");
    const void* src = nullptr;
    size_t need = 0;
    switch (type) {
        case ORT_OP_ATTR_INT: src = &a->value; need = sizeof(int64_t); break;
        case ORT_OP_ATTR_FLOAT: src = &a->fvalue; need = sizeof(float); break;
        case ORT_OP_ATTR_STRING: src = a->svalue.data(); need = a->svalue.size(); break;
        default: return mk_status(ORT_INVALID_ARGUMENT, "mock holds INT, FLOAT and STRING attributes");
    }
    *out = need;
    if (len < need || (need && !data)) return mk_status(ORT_INVALID_ARGUMENT, "buffer too small");
    if (need) std::memcpy(data, src, need);
    return nullptr;
}
OrtStatus* ORT_API_CALL m_GetValueInfoName(const OrtValueInfo* v, const char** out) NX {
    *out = v->name.c_str();
    return nullptr;
}
OrtStatus* ORT_API_CALL m_GetValueInfoTypeInfo(const OrtValueInfo* v, const OrtTypeInfo** out) NX {
    *out = &v->type;
    return nullptr;
}
OrtStatus* ORT_API_CALL m_CastTypeInfoToTensorInfo(const OrtTypeInfo* t,
                                                   const OrtTensorTypeAndShapeInfo** out) NX {
    *out = &t->tensor;
    return nullptr;
}
OrtStatus* ORT_API_CALL m_GetTensorElementType(const OrtTensorTypeAndShapeInfo* t,
                                               ONNXTensorElementDataType* out) NX {
    *out = (ONNXTensorElementDataType)t->elem;
    return nullptr;
}
OrtStatus* ORT_API_CALL m_GetDimensionsCount(const OrtTensorTypeAndShapeInfo* t, size_t* out) NX {
    *out = t->dims.size();
    return nullptr;
}
OrtStatus* ORT_API_CALL m_GetDimensions(const OrtTensorTypeAndShapeInfo* t, int64_t* d, size_t n) NX {
    for (size_t i = 0; i < n && i < t->dims.size(); ++i) d[i] = t->dims[i];
    return nullptr;
}
OrtStatus* ORT_API_CALL m_ValueInfo_IsConstantInitializer(const OrtValueInfo* v, bool* out) NX {
    *out = v->constant;
    return nullptr;
}

size_t elem_size(int32_t e) {
    switch (e) {
        case 1: return 4;
        case 2: return 1;
        case 10: return 2;
        default: return 1;
    }
}

// Initializer OrtValues handed out by ValueInfo_GetInitializerValue (owned by the host).
std::vector<std::unique_ptr<OrtValue>> g_init_values;

OrtStatus* ORT_API_CALL m_ValueInfo_GetInitializerValue(const OrtValueInfo* v, const OrtValue** out) NX {
    *out = nullptr;
    if (!v->constant) return nullptr;
    auto val = std::make_unique<OrtValue>();
    val->elem = v->type.tensor.elem;
    val->dims = v->type.tensor.dims;
    val->data = v->init.data();
    val->bytes = v->init.size();
    *out = val.get();
    g_init_values.push_back(std::move(val));
    return nullptr;
}
OrtStatus* ORT_API_CALL m_GetTensorData(const OrtValue* v, const void** out) NX {
    *out = v->data;
    return nullptr;
}
OrtStatus* ORT_API_CALL m_GetTensorMutableData(OrtValue* v, void** out) NX {
    *out = const_cast<void*>(v->data);
    return nullptr;
}
OrtStatus* ORT_API_CALL m_GetTensorSizeInBytes(const OrtValue* v, size_t* out) NX {
    *out = v->bytes;
    return nullptr;
}
OrtStatus* ORT_API_CALL m_GetTensorTypeAndShape(const OrtValue* v, OrtTensorTypeAndShapeInfo** out) NX {
    *out = new OrtTensorTypeAndShapeInfo{v->elem, v->dims};
    return nullptr;
}
void ORT_API_CALL m_ReleaseTensorTypeAndShapeInfo(OrtTensorTypeAndShapeInfo* t) NX { delete t; }

OrtStatus* ORT_API_CALL m_KernelContext_GetInputCount(const OrtKernelContext* c, size_t* out) NX {
    *out = c->inputs.size();
    return nullptr;
}
OrtStatus* ORT_API_CALL m_KernelContext_GetOutputCount(const OrtKernelContext* c, size_t* out) NX {
    *out = c->out_elem.size();
    return nullptr;
}
OrtStatus* ORT_API_CALL m_KernelContext_GetInput(const OrtKernelContext* c, size_t i, const OrtValue** out) NX {
    if (i >= c->inputs.size()) return mk_status(ORT_INVALID_ARGUMENT, "input index out of range");
    *out = c->inputs[i];
    return nullptr;
}
// Device-memory mode of the host: outputs are allocated with the EP's device allocator (as ORT
// does for an EP whose default memory device is its GPU); every such buffer is freed at reset.
OrtAllocator* g_out_alloc = nullptr;
const OrtMemoryDevice* g_out_md = nullptr;
std::vector<void*> g_dev_buffers;

OrtStatus* ORT_API_CALL m_KernelContext_GetOutput(OrtKernelContext* c, size_t i, const int64_t* dims,
                                                  size_t rank, OrtValue** out) NX {
    if (i >= c->out_elem.size()) return mk_status(ORT_INVALID_ARGUMENT, "output index out of range");
    auto v = std::make_unique<OrtValue>();
    v->elem = c->out_elem[i];
    v->dims.assign(dims, dims + rank);
    size_t n = 1;
    for (int64_t d : v->dims) n *= (size_t)d;
    v->bytes = n * elem_size(v->elem);
    if (g_out_alloc) {
        void* p = g_out_alloc->Alloc(g_out_alloc, v->bytes ? v->bytes : 1);
        if (!p) return mk_status(ORT_FAIL, "device allocator returned NULL");
        g_dev_buffers.push_back(p);
        v->data = p;
        v->md = g_out_md;
    } else {
        v->owned.assign(v->bytes + 16, 0xCD);   // poison: unwritten output is detectable
        v->data = v->owned.data();
    }
    *out = v.get();
    if (c->outputs.size() <= i) c->outputs.resize(i + 1);
    c->outputs[i] = std::move(v);
    return nullptr;
}

OrtStatus* ORT_API_CALL m_KernelContext_GetGPUComputeStream(const OrtKernelContext* c, void** out) NX {
    *out = c->stream;
    return nullptr;
}

void* ORT_API_CALL m_SyncStream_GetHandle(OrtSyncStream* s) NX {
    return s && s->impl ? s->impl->GetHandle(s->impl) : nullptr;
}

OrtHardwareDeviceType ORT_API_CALL m_HardwareDevice_Type(const OrtHardwareDevice* d) NX { return d->type; }
uint32_t ORT_API_CALL m_HardwareDevice_VendorId(const OrtHardwareDevice* d) NX { return d->vendor_id; }
uint32_t ORT_API_CALL m_HardwareDevice_DeviceId(const OrtHardwareDevice* d) NX { return d->device_id; }

void ORT_API_CALL m_CreateKeyValuePairs(OrtKeyValuePairs** out) NX { *out = new OrtKeyValuePairs(); }
void ORT_API_CALL m_AddKeyValuePair(OrtKeyValuePairs* kv, const char* k, const char* v) NX { kv->kv[k] = v; }
const char* ORT_API_CALL m_GetKeyValue(const OrtKeyValuePairs* kv, const char* k) NX {
    auto it = kv->kv.find(k);
    return it == kv->kv.end() ? nullptr : it->second.c_str();
}
void ORT_API_CALL m_ReleaseKeyValuePairs(OrtKeyValuePairs* kv) NX { delete kv; }

OrtStatus* ORT_API_CALL m_HasSessionConfigEntry(const OrtSessionOptions* so, const char* k, int* out) NX {
    *out = so->config.count(k) ? 1 : 0;
    return nullptr;
}
OrtStatus* ORT_API_CALL m_GetSessionConfigEntry(const OrtSessionOptions* so, const char* k, char* v,
                                                size_t* size) NX {
    auto it = so->config.find(k);
    if (it == so->config.end()) return mk_status(ORT_INVALID_ARGUMENT, "no such config entry");
    const size_t need = it->second.size() + 1;
    if (!v) {
        *size = need;
        return nullptr;
    }
    if (*size < need) {
        *size = need;
        return mk_status(ORT_INVALID_ARGUMENT, "buffer too small");
    }
    std::memcpy(v, it->second.c_str(), need);
    *size = need;
    return nullptr;
}

long g_live_mem_infos = 0;
OrtStatus* ORT_API_CALL m_CreateMemoryInfo_V2(const char* name, OrtMemoryInfoDeviceType type,
                                              uint32_t vendor, int32_t id, OrtDeviceMemoryType mem,
                                              size_t alignment, OrtAllocatorType at,
                                              OrtMemoryInfo** out) NX {
    *out = new OrtMemoryInfo{name ? name : "", OrtMemoryDevice{type, mem, vendor, id}, alignment, at};
    ++g_live_mem_infos;
    return nullptr;
}
void ORT_API_CALL m_ReleaseMemoryInfo(OrtMemoryInfo* mi) NX {
    if (!mi) return;
    --g_live_mem_infos;
    delete mi;
}

// ---- OrtEpApi implementation ------------------------------------------------------------------

OrtStatus* ORT_API_CALL m_EpDevice_AddAllocatorInfo(OrtEpDevice* d, const OrtMemoryInfo* mi) NX {
    if (!d || !mi) return mk_status(ORT_INVALID_ARGUMENT, "null AddAllocatorInfo argument");
    for (const OrtMemoryInfo*& e : d->alloc_infos)
        if (e->alloc_type == mi->alloc_type && e->dev.mem == mi->dev.mem) {
            e = mi;                 // "multiple calls for the same entry type replace"
            return nullptr;
        }
    d->alloc_infos.push_back(mi);
    return nullptr;
}
const OrtMemoryDevice* ORT_API_CALL m_MemoryInfo_GetMemoryDevice(const OrtMemoryInfo* mi) NX {
    return mi ? &mi->dev : nullptr;
}
const OrtMemoryDevice* ORT_API_CALL m_Value_GetMemoryDevice(const OrtValue* v) NX {
    return v ? v->md : nullptr;
}
bool ORT_API_CALL m_MemoryDevice_AreEqual(const OrtMemoryDevice* a, const OrtMemoryDevice* b) NX {
    return a && b && a->type == b->type && a->mem == b->mem && a->vendor == b->vendor && a->id == b->id;
}
OrtMemoryInfoDeviceType ORT_API_CALL m_MemoryDevice_GetDeviceType(const OrtMemoryDevice* d) NX { return d->type; }
OrtDeviceMemoryType ORT_API_CALL m_MemoryDevice_GetMemoryType(const OrtMemoryDevice* d) NX { return d->mem; }
uint32_t ORT_API_CALL m_MemoryDevice_GetVendorId(const OrtMemoryDevice* d) NX { return d->vendor; }
uint32_t ORT_API_CALL m_MemoryDevice_GetDeviceId(const OrtMemoryDevice* d) NX { return (uint32_t)d->id; }

std::vector<std::unique_ptr<OrtEpDevice>> g_ep_devices;

OrtStatus* ORT_API_CALL m_CreateEpDevice(OrtEpFactory* f, const OrtHardwareDevice* hw,
                                         const OrtKeyValuePairs* meta, const OrtKeyValuePairs*,
                                         OrtEpDevice** out) NX {
    auto d = std::make_unique<OrtEpDevice>();
    d->factory = f;
    d->hw = hw;
    if (meta) d->meta.kv = meta->kv;   // ORT copies the metadata
    *out = d.get();
    g_ep_devices.push_back(std::move(d));
    return nullptr;
}
OrtStatus* ORT_API_CALL m_AddNodesToFuse(OrtEpGraphSupportInfo* info, const OrtNode* const* nodes,
                                         size_t n, const OrtNodeFusionOptions* opts) NX {
    std::vector<const OrtNode*> group;
    for (size_t i = 0; i < n; ++i) {
        bool found = false;
        for (const OrtNode* g : info->graph->nodes) found = found || g == nodes[i];
        if (!found) return mk_status(ORT_INVALID_ARGUMENT, "node is not in the graph");
        group.push_back(nodes[i]);
    }
    info->groups.push_back(group);
    info->drop.push_back(opts ? opts->drop_constant_initializers : false);
    return nullptr;
}

OrtApi g_api;
OrtEpApi g_ep_api;
uint32_t g_offered_version = ORT_API_VERSION;

const OrtEpApi* ORT_API_CALL m_GetEpApi() NX { return &g_ep_api; }

const OrtApi* ORT_API_CALL m_GetApi(uint32_t v) NX {
    return (v >= 1 && v <= g_offered_version) ? &g_api : nullptr;
}
const char* ORT_API_CALL m_GetVersionString() NX { return "mock-1.28.0"; }
OrtApiBase g_base = {m_GetApi, m_GetVersionString};

void init_api() {
    std::memset(&g_api, 0, sizeof(g_api));
    std::memset(&g_ep_api, 0, sizeof(g_ep_api));
    g_api.CreateStatus = m_CreateStatus;
    g_api.GetErrorCode = m_GetErrorCode;
    g_api.GetErrorMessage = m_GetErrorMessage;
    g_api.ReleaseStatus = m_ReleaseStatus;
    g_api.Graph_GetNumNodes = m_Graph_GetNumNodes;
    g_api.Graph_GetNodes = m_Graph_GetNodes;
    g_api.Graph_GetParentNode = m_Graph_GetParentNode;
    g_api.Node_GetName = m_Node_GetName;
    g_api.Node_GetOperatorType = m_Node_GetOperatorType;
    g_api.Node_GetDomain = m_Node_GetDomain;
    g_api.Node_GetNumInputs = m_Node_GetNumInputs;
    g_api.Node_GetInputs = m_Node_GetInputs;
    g_api.Node_GetNumOutputs = m_Node_GetNumOutputs;
    g_api.Node_GetOutputs = m_Node_GetOutputs;
    g_api.Node_GetAttributeByName = m_Node_GetAttributeByName;
    g_api.ReadOpAttr = m_ReadOpAttr;
    g_api.GetValueInfoName = m_GetValueInfoName;
    g_api.GetValueInfoTypeInfo = m_GetValueInfoTypeInfo;
    g_api.CastTypeInfoToTensorInfo = m_CastTypeInfoToTensorInfo;
    g_api.GetTensorElementType = m_GetTensorElementType;
    g_api.GetDimensionsCount = m_GetDimensionsCount;
    g_api.GetDimensions = m_GetDimensions;
    g_api.ValueInfo_IsConstantInitializer = m_ValueInfo_IsConstantInitializer;
    g_api.ValueInfo_GetInitializerValue = m_ValueInfo_GetInitializerValue;
    g_api.GetTensorData = m_GetTensorData;
    g_api.GetTensorMutableData = m_GetTensorMutableData;
    g_api.GetTensorSizeInBytes = m_GetTensorSizeInBytes;
    g_api.GetTensorTypeAndShape = m_GetTensorTypeAndShape;
    g_api.ReleaseTensorTypeAndShapeInfo = m_ReleaseTensorTypeAndShapeInfo;
    g_api.KernelContext_GetInputCount = m_KernelContext_GetInputCount;
    g_api.KernelContext_GetOutputCount = m_KernelContext_GetOutputCount;
    g_api.KernelContext_GetInput = m_KernelContext_GetInput;
    g_api.KernelContext_GetOutput = m_KernelContext_GetOutput;
    g_api.KernelContext_GetGPUComputeStream = m_KernelContext_GetGPUComputeStream;
    g_api.SyncStream_GetHandle = m_SyncStream_GetHandle;
    g_api.HardwareDevice_Type = m_HardwareDevice_Type;
    g_api.HardwareDevice_VendorId = m_HardwareDevice_VendorId;
    g_api.HardwareDevice_DeviceId = m_HardwareDevice_DeviceId;
    g_api.CreateKeyValuePairs = m_CreateKeyValuePairs;
    g_api.AddKeyValuePair = m_AddKeyValuePair;
    g_api.GetKeyValue = m_GetKeyValue;
    g_api.ReleaseKeyValuePairs = m_ReleaseKeyValuePairs;
    g_api.HasSessionConfigEntry = m_HasSessionConfigEntry;
    g_api.GetSessionConfigEntry = m_GetSessionConfigEntry;
    g_api.GetEpApi = m_GetEpApi;
    g_api.CreateMemoryInfo_V2 = m_CreateMemoryInfo_V2;
    g_api.ReleaseMemoryInfo = m_ReleaseMemoryInfo;
    g_ep_api.CreateEpDevice = m_CreateEpDevice;
    g_ep_api.EpGraphSupportInfo_AddNodesToFuse = m_AddNodesToFuse;
    g_ep_api.EpDevice_AddAllocatorInfo = m_EpDevice_AddAllocatorInfo;
    g_ep_api.MemoryInfo_GetMemoryDevice = m_MemoryInfo_GetMemoryDevice;
    g_ep_api.Value_GetMemoryDevice = m_Value_GetMemoryDevice;
    g_ep_api.MemoryDevice_AreEqual = m_MemoryDevice_AreEqual;
    g_ep_api.MemoryDevice_GetDeviceType = m_MemoryDevice_GetDeviceType;
    g_ep_api.MemoryDevice_GetMemoryType = m_MemoryDevice_GetMemoryType;
    g_ep_api.MemoryDevice_GetVendorId = m_MemoryDevice_GetVendorId;
    g_ep_api.MemoryDevice_GetDeviceId = m_MemoryDevice_GetDeviceId;
}

// ---- host state ---------------------------------------------------------------------------------

using CreateFn = OrtStatus* (*)(const char*, const OrtApiBase*, const OrtLogger*, OrtEpFactory**,
                                size_t, size_t*);
using ReleaseFn = OrtStatus* (*)(OrtEpFactory*);

struct Group {
    std::unique_ptr<OrtGraph> graph;      // the island as its own graph
    std::unique_ptr<OrtNode> fused;       // the fused node ORT would create
    OrtNodeComputeInfo* info = nullptr;
};

struct Host {
    void* lib = nullptr;
    CreateFn create = nullptr;
    ReleaseFn release = nullptr;
    OrtEpFactory* factory = nullptr;
    std::vector<std::unique_ptr<OrtHardwareDevice>> hw;
    std::vector<OrtEpDevice*> ep_devices;
    OrtEp* ep = nullptr;
    OrtSessionOptions so;
    OrtLogger logger;
    std::map<std::string, std::unique_ptr<OrtValueInfo>> values;
    std::vector<std::unique_ptr<OrtNode>> nodes;
    OrtGraph graph;
    std::vector<Group> groups;
    std::vector<bool> drop;
    // host tensors for compute
    std::map<std::string, OrtValue> feeds;
    std::map<std::string, OrtValue> fetches;
    // device-memory mode
    OrtAllocator* dev_alloc = nullptr;
    OrtDataTransferImpl* dt = nullptr;
    const OrtMemoryDevice* dev_md = nullptr;
    // stream-aware EPs: the one stream of the session's device (ORT's default for one device)
    OrtSyncStream stream;
};
Host* g = nullptr;

int status_rc(OrtStatus* st) {
    if (!st) return 0;
    set_err("%s", st->msg.c_str());
    const int code = (int)st->code;
    m_ReleaseStatus(st);
    return code ? code : -1;
}

std::vector<std::string> split(const char* s, char sep) {
    std::vector<std::string> out;
    if (!s) return out;
    std::string cur;
    for (const char* p = s;; ++p) {
        if (*p == sep || *p == '\0') {
            out.push_back(cur);
            cur.clear();
            if (!*p) break;
        } else {
            cur += *p;
        }
    }
    return out;
}

}  // namespace

// ---- the C surface the tests drive -----------------------------------------------------------------

extern "C" {

const char* mock_last_error(void) { return g_err.c_str(); }
long mock_live_statuses(void) { return g_live_status; }
long mock_created_statuses(void) { return g_created_status; }
int mock_bad_status_release(void) { return g_bad_release ? 1 : 0; }

// dlopen the EP and call CreateEpFactories with an OrtApiBase offering versions <= api_version.
int mock_init(const char* ep_path, unsigned api_version) {
    init_api();
    g_offered_version = api_version;
    delete g;
    g = new Host();
    g->lib = dlopen(ep_path, RTLD_NOW | RTLD_LOCAL);
    if (!g->lib) {
        set_err("dlopen: %s", dlerror());
        return -1;
    }
    g->create = (CreateFn)dlsym(g->lib, "CreateEpFactories");
    g->release = (ReleaseFn)dlsym(g->lib, "ReleaseEpFactory");
    if (!g->create || !g->release) {
        set_err("the library does not export CreateEpFactories / ReleaseEpFactory");
        return -1;
    }
    OrtEpFactory* fs[4] = {nullptr, nullptr, nullptr, nullptr};
    size_t n = 0;
    int rc = status_rc(g->create("MI355XExecutionProvider", &g_base, &g->logger, fs, 4, &n));
    if (rc) return rc;
    if (n != 1 || !fs[0]) {
        set_err("expected one factory, got %zu", n);
        return -1;
    }
    g->factory = fs[0];
    return 0;
}

// Factory identity: returns the negotiated version the factory reports.
int mock_factory_info(char* name, size_t nlen, char* vendor, size_t vlen, unsigned* vendor_id,
                      unsigned* version) {
    if (!g || !g->factory) return -1;
    std::snprintf(name, nlen, "%s", g->factory->GetName(g->factory));
    std::snprintf(vendor, vlen, "%s", g->factory->GetVendor(g->factory));
    *vendor_id = g->factory->GetVendorId(g->factory);
    *version = g->factory->ort_version_supported;
    return 0;
}

// Offers `n_amd` AMD GPUs and `n_other` other GPUs; returns the number of EP devices advertised.
int mock_supported_devices(int n_amd, int n_other) {
    if (!g || !g->factory) return -1;
    g->hw.clear();
    for (int i = 0; i < n_amd; ++i)
        g->hw.push_back(std::make_unique<OrtHardwareDevice>(OrtHardwareDevice{OrtHardwareDeviceType_GPU, 0x1002, 0x75a3}));
    for (int i = 0; i < n_other; ++i)
        g->hw.push_back(std::make_unique<OrtHardwareDevice>(OrtHardwareDevice{OrtHardwareDeviceType_GPU, 0x10de, 0x2900}));
    g->hw.push_back(std::make_unique<OrtHardwareDevice>(OrtHardwareDevice{OrtHardwareDeviceType_CPU, 0x1022, 0}));
    std::vector<const OrtHardwareDevice*> hw;
    for (auto& h : g->hw) hw.push_back(h.get());
    OrtEpDevice* out[8] = {nullptr};
    size_t n = 99;
    int rc = status_rc(g->factory->GetSupportedDevices(g->factory, hw.data(), hw.size(), out, 8, &n));
    if (rc) return -rc;
    g->ep_devices.assign(out, out + n);
    return (int)n;
}

const char* mock_device_meta(int i, const char* key) {
    if (!g || i < 0 || i >= (int)g->ep_devices.size()) return nullptr;
    auto it = g->ep_devices[i]->meta.kv.find(key);
    return it == g->ep_devices[i]->meta.kv.end() ? nullptr : it->second.c_str();
}

void mock_session_option(const char* key, const char* value) {
    if (g) g->so.config[key] = value;
}

// CreateEp on advertised device `i` (or, with i < 0, on no metadata at all).
int mock_create_ep(int i) {
    if (!g || !g->factory) return -1;
    const OrtHardwareDevice* hw[1] = {g->hw.empty() ? nullptr : g->hw[0].get()};
    const OrtKeyValuePairs* meta[1] = {nullptr};
    if (i >= 0 && i < (int)g->ep_devices.size()) {
        hw[0] = g->ep_devices[i]->hw;
        meta[0] = &g->ep_devices[i]->meta;
    }
    OrtEp* ep = nullptr;
    int rc = status_rc(g->factory->CreateEp(g->factory, hw, meta, 1, &g->so, &g->logger, &ep));
    if (rc) return rc;
    if (!ep) {
        set_err("CreateEp returned success and no EP");
        return -1;
    }
    g->ep = ep;
    return 0;
}

int mock_create_ep_n(int num_devices) {
    if (!g || !g->factory) return -1;
    std::vector<const OrtHardwareDevice*> hw(num_devices, g->hw.empty() ? nullptr : g->hw[0].get());
    std::vector<const OrtKeyValuePairs*> meta(num_devices, nullptr);
    OrtEp* ep = nullptr;
    int rc = status_rc(g->factory->CreateEp(g->factory, hw.data(), meta.data(), num_devices, &g->so,
                                            &g->logger, &ep));
    if (!rc && ep) g->ep = ep;
    return rc;
}

const char* mock_ep_name(void) { return g && g->ep ? g->ep->GetName(g->ep) : nullptr; }

static void free_device_buffers() {
    if (g_out_alloc)
        for (void* p : g_dev_buffers) g_out_alloc->Free(g_out_alloc, p);
    g_dev_buffers.clear();
}

void mock_graph_reset(void) {
    if (!g) return;
    free_device_buffers();
    g->values.clear();
    g->nodes.clear();
    g->graph = OrtGraph();
    g->groups.clear();
    g->drop.clear();
    g->feeds.clear();
    g->fetches.clear();
}

// A graph value; `data` non-NULL makes it a constant initializer (its bytes are copied).
int mock_add_value(const char* name, int elem, int rank, const int64_t* dims, const void* data,
                   size_t bytes) {
    auto v = std::make_unique<OrtValueInfo>();
    v->name = name;
    v->type.tensor.elem = elem;
    v->type.tensor.dims.assign(dims, dims + rank);
    if (data) {
        v->constant = true;
        v->init.assign((const uint8_t*)data, (const uint8_t*)data + bytes);
    }
    g->values[name] = std::move(v);
    return 0;
}

// A node: inputs/outputs are comma-separated value names ("" = absent optional input);
// attrs is "K=64,N=32,bits=4"; "name:f=1.5" is a float and "name:s=swiglu" a string attribute.
int mock_add_node(const char* op, const char* domain, const char* name, const char* inputs,
                  const char* outputs, const char* int_attrs) {
    auto n = std::make_unique<OrtNode>();
    n->op_type = op;
    n->domain = domain;
    n->name = name;
    for (const std::string& s : split(inputs, ',')) {
        if (s.empty()) {
            n->inputs.push_back(nullptr);
            continue;
        }
        auto it = g->values.find(s);
        if (it == g->values.end()) {
            set_err("unknown value %s", s.c_str());
            return -1;
        }
        n->inputs.push_back(it->second.get());
    }
    for (const std::string& s : split(outputs, ',')) {
        if (s.empty()) {                                  // an absent optional output
            n->outputs.push_back(nullptr);
            continue;
        }
        auto it = g->values.find(s);
        if (it == g->values.end()) {
            set_err("unknown value %s", s.c_str());
            return -1;
        }
        n->outputs.push_back(it->second.get());
    }
    for (const std::string& kv : split(int_attrs, ',')) {
        if (kv.empty()) continue;
        const size_t eq = kv.find('=');
        std::string key = kv.substr(0, eq);
        const std::string val = kv.substr(eq + 1);
        OrtOpAttr a;
        const size_t colon = key.find(':');
        const char kind = colon == std::string::npos ? 'i' : key[colon + 1];
        a.name = key.substr(0, colon);
        if (kind == 'f') {
            a.type = ORT_OP_ATTR_FLOAT;
            a.fvalue = std::strtof(val.c_str(), nullptr);
        } else if (kind == 's') {
            a.type = ORT_OP_ATTR_STRING;
            a.svalue = val;
        } else {
            a.value = std::atoll(val.c_str());
        }
        n->attrs.push_back(a);
    }
    g->graph.nodes.push_back(n.get());
    g->nodes.push_back(std::move(n));
    return 0;
}

// GetCapability on the whole graph (nested=1 pretends it is a control-flow body).  Returns the
// number of fused groups; `out` receives "node[:drop|:keep];..." for the claimed nodes.
int mock_get_capability(int nested, char* out, size_t len) {
    if (!g || !g->ep) return -1;
    OrtNode parent_stub;
    g->graph.parent = nested ? &parent_stub : nullptr;
    OrtEpGraphSupportInfo info{&g->graph, {}, {}};
    int rc = status_rc(g->ep->GetCapability(g->ep, &g->graph, &info));
    g->graph.parent = nullptr;
    if (rc) return -rc;
    std::string s;
    g->groups.clear();
    g->drop = info.drop;
    for (size_t i = 0; i < info.groups.size(); ++i) {
        Group gr;
        gr.graph = std::make_unique<OrtGraph>();
        gr.fused = std::make_unique<OrtNode>();
        gr.fused->op_type = "MI355X_fused";
        gr.fused->domain = "";
        std::set<std::string> seen;
        for (const OrtNode* n : info.groups[i]) {
            gr.graph->nodes.push_back(const_cast<OrtNode*>(n));
            if (!s.empty()) s += ';';
            s += n->name + (info.drop[i] ? ":drop" : ":keep");
            gr.fused->name += n->name;
            for (OrtValueInfo* v : n->inputs) {
                if (!v || seen.count(v->name)) continue;
                if (v->constant && info.drop[i]) continue;   // ORT drops constant initializers
                seen.insert(v->name);
                gr.fused->inputs.push_back(v);
            }
            for (OrtValueInfo* v : n->outputs)
                if (v) gr.fused->outputs.push_back(v);       // ORT's fused node: real outputs only
        }
        g->groups.push_back(std::move(gr));
    }
    std::snprintf(out, len, "%s", s.c_str());
    return (int)info.groups.size();
}

// Compile every group; returns 0 or an error code.
int mock_compile(void) {
    if (!g || !g->ep) return -1;
    const size_t n = g->groups.size();
    std::vector<const OrtGraph*> graphs;
    std::vector<const OrtNode*> fused;
    for (auto& gr : g->groups) {
        graphs.push_back(gr.graph.get());
        fused.push_back(gr.fused.get());
    }
    std::vector<OrtNodeComputeInfo*> infos(n, reinterpret_cast<OrtNodeComputeInfo*>(0x1));
    std::vector<OrtNode*> ctx_nodes(n, reinterpret_cast<OrtNode*>(0x1));
    int rc = status_rc(g->ep->Compile(g->ep, graphs.data(), fused.data(), n, infos.data(), ctx_nodes.data()));
    for (size_t i = 0; i < n; ++i) {
        // On failure every slot must have been reset; on success every slot is a compute info.
        if (infos[i] == reinterpret_cast<OrtNodeComputeInfo*>(0x1)) {
            set_err("Compile left compute-info slot %zu unwritten", i);
            return -2;
        }
        if (ctx_nodes[i] == reinterpret_cast<OrtNode*>(0x1)) {
            set_err("Compile left EPContext slot %zu unwritten", i);
            return -2;
        }
        if (rc && infos[i]) {
            set_err("Compile failed but left compute info %zu set", i);
            return -2;
        }
        if (!rc) g->groups[i].info = infos[i];
    }
    return rc;
}

// Host tensor for a graph input (borrowed: the caller keeps `data` alive until compute ends).
int mock_feed(const char* name, int elem, int rank, const int64_t* dims, const void* data, size_t bytes) {
    OrtValue v;
    v.elem = elem;
    v.dims.assign(dims, dims + rank);
    v.data = data;
    v.bytes = bytes;
    g->feeds[name] = v;
    return 0;
}

// Runs group `i`'s compute (CreateState / Compute / ReleaseState); outputs go to fetches.
int mock_compute(int i) {
    if (!g || i < 0 || i >= (int)g->groups.size() || !g->groups[i].info) return -1;
    Group& gr = g->groups[i];
    OrtKernelContext ctx;
    std::vector<std::unique_ptr<OrtValue>> init_vals;
    for (OrtValueInfo* v : gr.fused->inputs) {
        auto it = g->feeds.find(v->name);
        auto ft = g->fetches.find(v->name);     // an earlier island's output, where it lives
        if (it != g->feeds.end()) {
            ctx.inputs.push_back(&it->second);
        } else if (ft != g->fetches.end()) {
            ctx.inputs.push_back(&ft->second);
        } else if (v->constant) {
            auto val = std::make_unique<OrtValue>();
            val->elem = v->type.tensor.elem;
            val->dims = v->type.tensor.dims;
            val->data = v->init.data();
            val->bytes = v->init.size();
            ctx.inputs.push_back(val.get());
            init_vals.push_back(std::move(val));
        } else {
            set_err("no feed for %s", v->name.c_str());
            return -1;
        }
    }
    for (OrtValueInfo* v : gr.fused->outputs) ctx.out_elem.push_back(v->type.tensor.elem);
    ctx.stream = g->stream.impl ? g->stream.impl->GetHandle(g->stream.impl) : nullptr;
    OrtNodeComputeInfo* info = gr.info;
    void* state = nullptr;
    int rc = 0;
    if (info->CreateState) rc = status_rc(info->CreateState(info, nullptr, &state));
    if (rc) return rc;
    rc = status_rc(info->Compute(info, state, &ctx));
    if (info->ReleaseState) info->ReleaseState(info, state);
    if (rc) return rc;
    for (size_t o = 0; o < ctx.outputs.size() && o < gr.fused->outputs.size(); ++o) {
        if (!ctx.outputs[o]) continue;
        OrtValue& dst = g->fetches[gr.fused->outputs[o]->name];
        dst.elem = ctx.outputs[o]->elem;
        dst.dims = ctx.outputs[o]->dims;
        dst.owned = ctx.outputs[o]->owned;
        dst.bytes = ctx.outputs[o]->bytes;
        dst.md = ctx.outputs[o]->md;
        dst.data = dst.md == &kHostDevice ? (const void*)dst.owned.data() : ctx.outputs[o]->data;
    }
    return 0;
}

// Copies a fetched output; returns its rank (dims written to `dims`), or -1.
int mock_fetch(const char* name, void* dst, size_t bytes, int64_t* dims, int max_rank) {
    auto it = g->fetches.find(name);
    if (it == g->fetches.end()) {
        set_err("no output %s", name);
        return -1;
    }
    const OrtValue& v = it->second;
    if (bytes < v.bytes) {
        set_err("destination holds %zu bytes, output has %zu", bytes, v.bytes);
        return -1;
    }
    if (v.md != &kHostDevice) {
        if (!g->dt) {
            set_err("a device output and no data transfer");
            return -1;
        }
        OrtValue h;
        h.elem = v.elem;
        h.dims = v.dims;
        h.data = dst;
        h.bytes = v.bytes;
        const OrtValue* src[1] = {&v};
        OrtValue* dsts[1] = {&h};
        OrtSyncStream* st[1] = {&g->stream};
        int rc = status_rc(g->dt->CopyTensors(g->dt, src, dsts, g->stream.impl ? st : nullptr, 1));
        if (rc) return -1;
    } else {
        std::memcpy(dst, v.data, v.bytes);
    }
    for (int d = 0; d < (int)v.dims.size() && d < max_rank; ++d) dims[d] = v.dims[d];
    return (int)v.dims.size();
}

// ---- device memory (MI355X_EP_DEVICE_MEMORY) --------------------------------------------------

long mock_live_memory_infos(void) { return g_live_mem_infos; }

// Allocator infos EP device `i` registered with EpDevice_AddAllocatorInfo; `type`, `vendor`,
// `id` receive the first one's memory device.
int mock_allocator_infos(int i, int* type, unsigned* vendor, int* id) {
    if (!g || i < 0 || i >= (int)g->ep_devices.size()) return -1;
    const auto& v = g->ep_devices[i]->alloc_infos;
    if (!v.empty()) {
        *type = (int)v[0]->dev.type;
        *vendor = v[0]->dev.vendor;
        *id = v[0]->dev.id;
    }
    return (int)v.size();
}

// CreateAllocator for a memory info of the given description: 1 = an allocator came back (it
// is released again), 0 = declined, < 0 = an error status.
int mock_create_allocator_for(int type, unsigned vendor, int id, int mem) {
    if (!g || !g->factory) return -1;
    OrtMemoryInfo mi{"probe", OrtMemoryDevice{(OrtMemoryInfoDeviceType)type, (OrtDeviceMemoryType)mem,
                                              vendor, id}, 256, OrtDeviceAllocator};
    OrtAllocator* a = reinterpret_cast<OrtAllocator*>(0x1);
    int rc = status_rc(g->factory->CreateAllocator(g->factory, &mi, nullptr, &a));
    if (a == reinterpret_cast<OrtAllocator*>(0x1)) {
        set_err("CreateAllocator left its out-parameter unwritten");
        return -2;
    }
    if (rc) return -rc;
    if (!a) return 0;
    g->factory->ReleaseAllocator(g->factory, a);
    return 1;
}

// CanCopy between two memory devices: 1 / 0, or -1 when the factory offers no data transfer.
int mock_can_copy(int stype, unsigned svendor, int dtype, unsigned dvendor) {
    if (!g || !g->factory) return -1;
    OrtDataTransferImpl* dt = nullptr;
    if (status_rc(g->factory->CreateDataTransfer(g->factory, &dt))) return -2;
    if (!dt) return -1;
    OrtMemoryDevice s{(OrtMemoryInfoDeviceType)stype, OrtDeviceMemoryType_DEFAULT, svendor, 0};
    OrtMemoryDevice d{(OrtMemoryInfoDeviceType)dtype, OrtDeviceMemoryType_DEFAULT, dvendor, 0};
    const bool ok = dt->CanCopy(dt, &s, &d);
    dt->Release(dt);
    return ok ? 1 : 0;
}

// The EP's GetDefaultMemoryDevice: 1 = a device (written out), 0 = NULL, -2 = slot not set.
int mock_default_memory_device(int* type, unsigned* vendor, int* id) {
    if (!g || !g->ep) return -1;
    if (!g->ep->GetDefaultMemoryDevice) return -2;
    const OrtMemoryDevice* md = nullptr;
    int rc = status_rc(g->ep->GetDefaultMemoryDevice(g->ep, &md));
    if (rc) return -rc;
    if (!md) return 0;
    *type = (int)md->type;
    *vendor = md->vendor;
    *id = md->id;
    return 1;
}

// Device-memory session set-up the way ORT does it for an EP whose default memory device is its
// GPU: the factory's allocator for EP device `i`'s registered memory info, its data transfer,
// and outputs allocated in device memory.
int mock_device_io_setup(int i) {
    if (!g || !g->factory || i < 0 || i >= (int)g->ep_devices.size()) return -1;
    if (g->ep_devices[i]->alloc_infos.empty()) {
        set_err("EP device %d registered no allocator info", i);
        return -1;
    }
    const OrtMemoryInfo* mi = g->ep_devices[i]->alloc_infos[0];
    OrtAllocator* a = nullptr;
    int rc = status_rc(g->factory->CreateAllocator(g->factory, mi, nullptr, &a));
    if (rc) return rc;
    if (!a) {
        set_err("CreateAllocator declined the EP's own memory info");
        return -1;
    }
    OrtDataTransferImpl* dt = nullptr;
    rc = status_rc(g->factory->CreateDataTransfer(g->factory, &dt));
    if (rc || !dt) {
        g->factory->ReleaseAllocator(g->factory, a);
        if (!rc) set_err("no data transfer");
        return rc ? rc : -1;
    }
    g->dev_alloc = a;
    g->dt = dt;
    g->dev_md = &mi->dev;
    g_out_alloc = a;
    g_out_md = &mi->dev;
    return 0;
}

// A graph input placed in device memory: allocated with the EP's allocator and filled from
// `data` through the EP's data transfer (as ORT's MemcpyFromHost would).
int mock_feed_device(const char* name, int elem, int rank, const int64_t* dims, const void* data,
                     size_t bytes) {
    if (!g || !g->dev_alloc || !g->dt) {
        set_err("device I/O is not set up");
        return -1;
    }
    void* p = g->dev_alloc->Alloc(g->dev_alloc, bytes ? bytes : 1);
    if (!p) {
        set_err("device allocation failed");
        return -1;
    }
    g_dev_buffers.push_back(p);
    OrtValue h;
    h.elem = elem;
    h.dims.assign(dims, dims + rank);
    h.data = data;
    h.bytes = bytes;
    OrtValue d = h;
    d.data = p;
    d.md = g->dev_md;
    const OrtValue* src[1] = {&h};
    OrtValue* dst[1] = {&d};
    OrtSyncStream* st[1] = {&g->stream};
    int rc = status_rc(g->dt->CopyTensors(g->dt, src, dst, g->stream.impl ? st : nullptr, 1));
    if (rc) return rc;
    g->feeds[name] = d;
    return 0;
}

// Stream set-up the way ORT does it for a stream-aware EP (after mock_device_io_setup): one
// OrtSyncStreamImpl for the device's memory, created through CreateSyncStreamForDevice; computes
// and copies then carry it.  Returns 1 (stream created), 0 (the factory is not stream-aware),
// or an error code.
int mock_stream_setup(void) {
    if (!g || !g->factory || !g->dev_md) {
        set_err("device I/O is not set up");
        return -1;
    }
    if (!g->factory->IsStreamAware || !g->factory->IsStreamAware(g->factory)) return 0;
    OrtSyncStreamImpl* impl = nullptr;
    int rc = status_rc(g->factory->CreateSyncStreamForDevice(g->factory, g->dev_md, nullptr, &impl));
    if (rc) return rc;
    if (!impl) {
        set_err("a stream-aware factory created no stream");
        return -1;
    }
    g->stream.impl = impl;
    return 1;
}

// IsStreamAware of the loaded factory (-1 without one).
int mock_is_stream_aware(void) {
    if (!g || !g->factory) return -1;
    return g->factory->IsStreamAware && g->factory->IsStreamAware(g->factory) ? 1 : 0;
}

// The stream's native handle (null without a stream).
void* mock_stream_handle(void) {
    return g && g->stream.impl ? g->stream.impl->GetHandle(g->stream.impl) : nullptr;
}

// What ORT does when a run ends: OnSessionRunEnd on the run's stream.
int mock_run_end(void) {
    if (!g || !g->stream.impl) return 0;
    return status_rc(g->stream.impl->OnSessionRunEnd(g->stream.impl));
}

// A notification from the stream, activated, waited on by the stream itself and by the host,
// released (ORT's cross-stream and stream-to-host synchronisation).
int mock_notification_roundtrip(void) {
    if (!g || !g->stream.impl) {
        set_err("no stream");
        return -1;
    }
    OrtSyncStreamImpl* impl = g->stream.impl;
    OrtSyncNotificationImpl* n = nullptr;
    int rc = status_rc(impl->CreateNotification(impl, &n));
    if (rc) return rc;
    if (!n) {
        set_err("CreateNotification returned no notification");
        return -1;
    }
    rc = status_rc(n->Activate(n));
    if (!rc) rc = status_rc(n->WaitOnDevice(n, &g->stream));
    if (!rc) rc = status_rc(n->WaitOnHost(n));
    if (!rc) rc = status_rc(impl->Flush(impl));
    n->Release(n);
    return rc;
}

// Releases compute infos, the EP and the factory (in ORT's order) and unloads the library.
int mock_shutdown(void) {
    if (!g) return 0;
    if (g->stream.impl) g->stream.impl->Release(g->stream.impl);   // drains its work first
    g->stream.impl = nullptr;
    free_device_buffers();
    if (g->dev_alloc && g->factory) g->factory->ReleaseAllocator(g->factory, g->dev_alloc);
    g->dev_alloc = nullptr;
    g_out_alloc = nullptr;
    g_out_md = nullptr;
    if (g->dt) g->dt->Release(g->dt);
    g->dt = nullptr;
    if (g->ep) {
        std::vector<OrtNodeComputeInfo*> infos;
        for (auto& gr : g->groups)
            if (gr.info) infos.push_back(gr.info);
        if (!infos.empty()) g->ep->ReleaseNodeComputeInfos(g->ep, infos.data(), infos.size());
        g->factory->ReleaseEp(g->factory, g->ep);
        g->ep = nullptr;
    }
    int rc = 0;
    if (g->factory) rc = status_rc(g->release(g->factory));
    g->factory = nullptr;
    g_init_values.clear();
    g_ep_devices.clear();
    // The library stays loaded: HIP's runtime does not support being unloaded mid-process.
    delete g;
    g = nullptr;
    return rc;
}

}  // extern "C"
