// ONNX Runtime plugin execution provider for com.microsoft::MatMulNBits on MI355X (gfx950).
//
// The exported surface is the plugin-EP ABI a stock ORT resolves by name (include/
// onnxruntime_mi355x_ep.h): CreateEpFactories / ReleaseEpFactory.  Behind it:
//   factory   OrtEpFactory: advertises each gfx950 GPU as an OrtEpDevice, creates one OrtEp per
//             session bound to exactly one device (reference: rust/src/factory.rs:57-118,
//             :189-480, :835-940).
//   ep        OrtEp: GetCapability claims MatMulNBits nodes (predicate in claim.hpp, reference
//             rust/src/ops/quant.rs:110-203; fused one node per island, reference
//             rust/src/ep.rs:1514-1537), Compile builds one compute info per island and uploads
//             constant B / scales / zero_points to HBM once (the reference uploads them at the
//             first Compute, keyed by host pointer, rust/src/vk/session.rs:1633-1700), and
//             Compute stages A in, launches one HIP kernel and copies Y out
//             (rust/src/ep.rs:2538-2716, rust/src/vk/session.rs:1036).
// With MI355X_EP_DEVICE_MEMORY=1 (off by default, as the reference's
// ONNXRUNTIME_EP_VULKAN_DEVICE_MEMORY, rust/src/factory.rs:487-504) the EP also advertises its
// HBM to ORT: an OrtAllocator over hipMalloc per device, an OrtDataTransferImpl for host <-> HBM
// copies, and the default memory device, so ORT keeps A and Y in HBM and Compute launches on
// device pointers with no staging (reference: rust/src/factory.rs:1043-1285, allocator.rs,
// transfer.rs).
// Every vtable entry is wrapped so that a C++ exception becomes an OrtStatus and never unwinds
// into ORT (the reference's guard_ffi_*, rust/src/lib.rs:99-206).  A Compute failure is always
// reported as a status; nothing is recomputed on the CPU.
#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cctype>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>
#include <vector>

#include "onnxruntime_c_api.h"   // also declares the plugin-EP ABI (onnxruntime_ep_c_api.h)

#include "claim.hpp"
#include "mnb_hip.h"
#include "onnxruntime_mi355x_ep.h"

#define MI355X_EXPORT extern "C" __attribute__((visibility("default")))

namespace mi355x_ep {
namespace {

constexpr uint32_t kVersionBuilt = ORT_API_VERSION;
constexpr uint32_t kVersionMin = MI355X_EP_ORT_API_VERSION_MIN;
static_assert(ORT_API_VERSION == MI355X_EP_ORT_API_VERSION_BUILT,
              "ORT headers declare a different ORT_API_VERSION than this EP was written for");
constexpr uint32_t kAmdVendorId = 0x1002;
const char* const kEpName = MI355X_EP_NAME;
const char* const kEpVendor = "onnxruntime-ep-mi355x";
const char* const kEpVersion = "0.28.0";
const char* const kMetaDeviceIndex = "mi355x.hip_device_index";

std::atomic<uint64_t> g_compute_count{0};

// ---- errors ------------------------------------------------------------------------------

struct EpError : std::runtime_error {
    OrtErrorCode code;
    EpError(OrtErrorCode c, const std::string& m) : std::runtime_error(m), code(c) {}
};

[[noreturn]] void fail(OrtErrorCode code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    throw EpError(code, buf);
}

std::string status_text(const OrtApi* api, OrtStatus* st) {
    const char* m = api->GetErrorMessage(st);
    std::string s = m ? m : "<null message>";
    api->ReleaseStatus(st);
    return s;
}

// Turns an ORT call's status into an exception (releasing the status exactly once).
void ort_check(const OrtApi* api, OrtStatus* st, const char* what) {
    if (!st) return;
    const OrtErrorCode code = api->GetErrorCode(st);
    const std::string msg = status_text(api, st);
    throw EpError(code, std::string(what) + ": " + msg);
}
#define ORT_OK(api, call) ort_check((api), (api)->call, #call)

void mnb_ok(int rc, const char* what) {
    if (rc == MNB_OK) return;
    const OrtErrorCode code = rc == MNB_ERR_INVALID ? ORT_INVALID_ARGUMENT : ORT_EP_FAIL;
    throw EpError(code, std::string(what) + ": " + mnb_last_error());
}

// The strip-major copy of a node's weights (ep.strip_major_weights).  Nodes the batched decode
// kernel never runs keep ORT's layout only; any other failure fails the upload.
void prepack_weights(mnb_weights* w) {
    const int rc = mnb_weights_prepack(w, nullptr);
    if (rc != MNB_ERR_UNSUPPORTED) mnb_ok(rc, "strip-major copy of MatMulNBits weights");
}

OrtStatus* to_status(const OrtApi* api, OrtErrorCode code, const std::string& msg) {
    if (!api) return nullptr;
    return api->CreateStatus(code, msg.c_str());
}

// Runs `f`, converting any exception into an OrtStatus for ORT.
template <typename F>
OrtStatus* guarded(const OrtApi* api, const char* where, F&& f) {
    try {
        f();
        return nullptr;
    } catch (const EpError& e) {
        return to_status(api, e.code, std::string(kEpName) + " " + where + ": " + e.what());
    } catch (const std::bad_alloc&) {
        return to_status(api, ORT_EP_FAIL, std::string(kEpName) + " " + where + ": out of memory");
    } catch (const std::exception& e) {
        return to_status(api, ORT_EP_FAIL, std::string(kEpName) + " " + where + ": " + e.what());
    } catch (...) {
        return to_status(api, ORT_EP_FAIL, std::string(kEpName) + " " + where + ": unknown error");
    }
}

bool env_flag(const char* name) {
    const char* v = std::getenv(name);
    return v && *v && std::strcmp(v, "0") != 0;
}

// The one reader of MI355X_EP_DEVICE_MEMORY.  The mode ships off, so only an explicit "on"
// spelling enables it; anything else (including typos of "off") leaves the host-I/O path.
bool device_memory_requested() {
    const char* v = std::getenv("MI355X_EP_DEVICE_MEMORY");
    if (!v) return false;
    std::string s;
    for (const char* p = v; *p; ++p)
        if (!std::isspace((unsigned char)*p)) s += (char)std::tolower((unsigned char)*p);
    return s == "1" || s == "true" || s == "yes" || s == "on";
}

void claim_log(const char* fmt, ...) {
    if (!env_flag("MI355X_EP_CLAIM_DEBUG")) return;
    va_list ap;
    va_start(ap, fmt);
    std::fprintf(stderr, "[mi355x-ep] ");
    std::vfprintf(stderr, fmt, ap);
    std::fprintf(stderr, "\n");
    va_end(ap);
}

// ---- reading the ORT graph ------------------------------------------------------------------

std::string node_string(const OrtApi* api, const OrtNode* node,
                        OrtStatus* (*getter)(const OrtNode*, const char**)) {
    const char* s = nullptr;
    OrtStatus* st = getter(node, &s);
    if (st) {
        api->ReleaseStatus(st);
        return {};
    }
    return s ? s : "";
}

std::string value_name(const OrtApi* api, const OrtValueInfo* vi) {
    if (!vi) return {};
    const char* s = nullptr;
    ORT_OK(api, GetValueInfoName(vi, &s));
    return s ? s : "";
}

std::vector<const OrtValueInfo*> node_inputs(const OrtApi* api, const OrtNode* node) {
    size_t n = 0;
    ORT_OK(api, Node_GetNumInputs(node, &n));
    std::vector<const OrtValueInfo*> v(n, nullptr);
    if (n) ORT_OK(api, Node_GetInputs(node, v.data(), n));
    return v;
}

std::vector<const OrtValueInfo*> node_outputs(const OrtApi* api, const OrtNode* node) {
    size_t n = 0;
    ORT_OK(api, Node_GetNumOutputs(node, &n));
    std::vector<const OrtValueInfo*> v(n, nullptr);
    if (n) ORT_OK(api, Node_GetOutputs(node, v.data(), n));
    return v;
}

InputFacts input_facts(const OrtApi* api, const OrtValueInfo* vi) {
    InputFacts f;
    if (!vi) return f;
    f.present = true;
    const OrtTypeInfo* ti = nullptr;
    ORT_OK(api, GetValueInfoTypeInfo(vi, &ti));
    if (ti) {
        const OrtTensorTypeAndShapeInfo* tsi = nullptr;
        ORT_OK(api, CastTypeInfoToTensorInfo(ti, &tsi));
        if (tsi) {
            ONNXTensorElementDataType et = ONNX_TENSOR_ELEMENT_DATA_TYPE_UNDEFINED;
            ORT_OK(api, GetTensorElementType(tsi, &et));
            f.elem_type = (int32_t)et;
            size_t rank = 0;
            ORT_OK(api, GetDimensionsCount(tsi, &rank));
            f.dims.assign(rank, 0);
            if (rank) ORT_OK(api, GetDimensions(tsi, f.dims.data(), rank));
            f.has_shape = true;
        }
    }
    bool is_const = false;
    OrtStatus* st = api->ValueInfo_IsConstantInitializer(vi, &is_const);
    if (st) {
        api->ReleaseStatus(st);
        is_const = false;
    }
    f.constant = is_const;
    return f;
}

bool int_attr(const OrtApi* api, const OrtNode* node, const char* name, int64_t* out) {
    const OrtOpAttr* attr = nullptr;
    OrtStatus* st = api->Node_GetAttributeByName(node, name, &attr);
    if (st) {
        api->ReleaseStatus(st);
        return false;
    }
    if (!attr) return false;
    int64_t v = 0;
    size_t got = 0;
    st = api->ReadOpAttr(attr, ORT_OP_ATTR_INT, &v, sizeof(v), &got);
    if (st) {
        api->ReleaseStatus(st);
        return false;
    }
    *out = v;
    return true;
}

NodeFacts node_facts(const OrtApi* api, const OrtNode* node) {
    NodeFacts f;
    f.op_type = node_string(api, node, api->Node_GetOperatorType);
    f.domain = node_string(api, node, api->Node_GetDomain);
    if (!is_matmul_nbits(f)) return f;
    for (const OrtValueInfo* vi : node_inputs(api, node)) f.inputs.push_back(input_facts(api, vi));
    f.num_outputs = node_outputs(api, node).size();
    f.has_k = int_attr(api, node, "K", &f.k);
    f.has_n = int_attr(api, node, "N", &f.n);
    f.has_bits = int_attr(api, node, "bits", &f.bits);
    f.has_block_size = int_attr(api, node, "block_size", &f.block_size);
    f.has_accuracy_level = int_attr(api, node, "accuracy_level", &f.accuracy_level);
    return f;
}

bool float_attr(const OrtApi* api, const OrtNode* node, const char* name, float* out) {
    const OrtOpAttr* attr = nullptr;
    OrtStatus* st = api->Node_GetAttributeByName(node, name, &attr);
    if (st) {
        api->ReleaseStatus(st);
        return false;
    }
    if (!attr) return false;
    float v = 0.f;
    size_t got = 0;
    st = api->ReadOpAttr(attr, ORT_OP_ATTR_FLOAT, &v, sizeof(v), &got);
    if (st) {
        api->ReleaseStatus(st);
        return false;
    }
    *out = v;
    return true;
}

// ReadOpAttr reports the byte count a string needs when the buffer is too small; the string is
// read with a buffer of that size (no terminator is written).
bool string_attr(const OrtApi* api, const OrtNode* node, const char* name, std::string* out) {
    const OrtOpAttr* attr = nullptr;
    OrtStatus* st = api->Node_GetAttributeByName(node, name, &attr);
    if (st) {
        api->ReleaseStatus(st);
        return false;
    }
    if (!attr) return false;
    size_t need = 0;
    st = api->ReadOpAttr(attr, ORT_OP_ATTR_STRING, nullptr, 0, &need);
    if (st) api->ReleaseStatus(st);
    std::string buf(need, '\0');
    size_t got = 0;
    st = api->ReadOpAttr(attr, ORT_OP_ATTR_STRING, need ? &buf[0] : nullptr, need, &got);
    if (st) {
        api->ReleaseStatus(st);
        return false;
    }
    buf.resize(std::min(got, need));
    *out = buf;
    return true;
}

QmoeFacts qmoe_facts(const OrtApi* api, const OrtNode* node) {
    QmoeFacts f;
    f.op_type = node_string(api, node, api->Node_GetOperatorType);
    f.domain = node_string(api, node, api->Node_GetDomain);
    if (!is_qmoe(f.op_type, f.domain)) return f;
    for (const OrtValueInfo* vi : node_inputs(api, node)) f.inputs.push_back(input_facts(api, vi));
    f.num_outputs = node_outputs(api, node).size();
    f.has_k = int_attr(api, node, "k", &f.k);
    string_attr(api, node, "activation_type", &f.activation_type);
    int_attr(api, node, "normalize_routing_weights", &f.normalize_routing_weights);
    int_attr(api, node, "use_sparse_mixer", &f.use_sparse_mixer);
    int_attr(api, node, "swiglu_fusion", &f.swiglu_fusion);
    int_attr(api, node, "expert_weight_bits", &f.expert_weight_bits);
    int_attr(api, node, "block_size", &f.block_size);
    int_attr(api, node, "weights_prepacked", &f.weights_prepacked);
    f.has_quant_type = string_attr(api, node, "quant_type", &f.quant_type);
    float_attr(api, node, "activation_alpha", &f.activation_alpha);
    float_attr(api, node, "activation_beta", &f.activation_beta);
    f.has_swiglu_limit = float_attr(api, node, "swiglu_limit", &f.swiglu_limit);
    return f;
}

NormFacts norm_facts(const OrtApi* api, const OrtNode* node) {
    NormFacts f;
    f.op_type = node_string(api, node, api->Node_GetOperatorType);
    f.domain = node_string(api, node, api->Node_GetDomain);
    if (!is_skip_norm(f.op_type, f.domain) && !is_plain_norm(f.op_type, f.domain)) return f;
    for (const OrtValueInfo* vi : node_inputs(api, node)) f.inputs.push_back(input_facts(api, vi));
    for (const OrtValueInfo* vi : node_outputs(api, node)) f.outputs.push_back(vi != nullptr);
    f.has_axis = int_attr(api, node, "axis", &f.axis);
    f.has_stash_type = int_attr(api, node, "stash_type", &f.stash_type);
    float_attr(api, node, "epsilon", &f.epsilon);
    return f;
}

GqaFacts gqa_facts(const OrtApi* api, const OrtNode* node) {
    GqaFacts f;
    f.op_type = node_string(api, node, api->Node_GetOperatorType);
    f.domain = node_string(api, node, api->Node_GetDomain);
    if (!is_gqa(f.op_type, f.domain)) return f;
    for (const OrtValueInfo* vi : node_inputs(api, node)) f.inputs.push_back(input_facts(api, vi));
    for (const OrtValueInfo* vi : node_outputs(api, node)) f.outputs.push_back(input_facts(api, vi));
    f.has_num_heads = int_attr(api, node, "num_heads", &f.num_heads);
    f.has_kv_num_heads = int_attr(api, node, "kv_num_heads", &f.kv_num_heads);
    int_attr(api, node, "local_window_size", &f.local_window_size);
    int_attr(api, node, "do_rotary", &f.do_rotary);
    int_attr(api, node, "rotary_interleaved", &f.rotary_interleaved);
    int_attr(api, node, "smooth_softmax", &f.smooth_softmax);
    int_attr(api, node, "qk_output", &f.qk_output);
    int_attr(api, node, "kv_cache_bit_width", &f.kv_cache_bit_width);
    int_attr(api, node, "rotary_embedding_dim", &f.rotary_embedding_dim);
    float_attr(api, node, "softcap", &f.softcap);
    f.has_scale = float_attr(api, node, "scale", &f.scale);
    string_attr(api, node, "k_quant_type", &f.k_quant_type);
    string_attr(api, node, "v_quant_type", &f.v_quant_type);
    return f;
}

// Session option `key` (ORT prefixes EP options with "ep.<name>."; both spellings are read).
bool session_option(const OrtApi* api, const OrtSessionOptions* so, const std::string& key,
                    std::string* value) {
    if (!so) return false;
    for (const std::string& k : {key, "ep." + std::string(kEpName) + "." + key.substr(3)}) {
        int has = 0;
        OrtStatus* st = api->HasSessionConfigEntry(so, k.c_str(), &has);
        if (st) {
            api->ReleaseStatus(st);
            continue;
        }
        if (!has) continue;
        size_t size = 0;
        st = api->GetSessionConfigEntry(so, k.c_str(), nullptr, &size);
        if (st) {
            api->ReleaseStatus(st);
            continue;
        }
        std::string buf(size, '\0');
        st = api->GetSessionConfigEntry(so, k.c_str(), &buf[0], &size);
        if (st) {
            api->ReleaseStatus(st);
            continue;
        }
        buf.resize(std::strlen(buf.c_str()));
        *value = buf;
        return true;
    }
    return false;
}

// ---- objects ORT holds ------------------------------------------------------------------------

struct Factory;
struct Ep;

// One claimed MatMulNBits node after Compile.
struct NodeKernel {
    mnb_problem prob{};             // m filled per call
    size_t fused_a = 0;             // fused-node input index of A
    // Fused-node input index of B / scales / zero_points, or SIZE_MAX when they were dropped
    // (constant initializers uploaded at Compile).
    size_t fused_w[3] = {SIZE_MAX, SIZE_MAX, SIZE_MAX};
    bool resident = false;          // weights uploaded at Compile
    mnb_weights* weights = nullptr; // resident weights, or the last per-call upload
    std::mutex mu;
    std::string name;
    // QMoE node (qmoe set): x and router logits by fused-input index, expert tensors resident.
    bool qmoe = false;
    mnb_qmoe_problem qprob{};
    size_t fused_router = SIZE_MAX;
    int32_t router_elem = 0;
    mnb_qmoe_weights* qweights = nullptr;
    // RMSNorm node (norm set): skip by fused-input index; y and the residual sum by fused-output
    // index (SIZE_MAX when the node has no such output).
    bool norm = false;
    mnb_rmsnorm_problem nprob{};
    size_t fused_skip = SIZE_MAX;
    size_t fused_y = SIZE_MAX, fused_sum = SIZE_MAX;
    mnb_rmsnorm_weights* nweights = nullptr;
    // GroupQueryAttention node (gqa set): fused-input index of qkv (fused_a), past_key,
    // past_value, seqlens_k, cos_cache, sin_cache (the caches SIZE_MAX when resident) and
    // fused-output index of the output, present_key and present_value.
    bool gqa = false;
    mnb_gqa_problem gprob{};        // node constants; shapes filled per call
    int64_t gqa_packed = 0;
    int64_t gqa_present_len = -1;   // declared present length, or -1 (growing: past + S)
    size_t gqa_in[6] = {SIZE_MAX, SIZE_MAX, SIZE_MAX, SIZE_MAX, SIZE_MAX, SIZE_MAX};
    size_t gqa_out[3] = {SIZE_MAX, SIZE_MAX, SIZE_MAX};
    mnb_gqa_caches* gcaches = nullptr;

    ~NodeKernel() {
        if (weights) mnb_weights_release(weights);
        if (qweights) mnb_qmoe_weights_release(qweights);
        if (nweights) mnb_rmsnorm_weights_release(nweights);
        if (gcaches) mnb_gqa_caches_release(gcaches);
    }
};

struct ComputeInfo {
    OrtNodeComputeInfo base;        // first member: ORT's pointer is this object's pointer
    Ep* ep = nullptr;
    std::unique_ptr<NodeKernel> kernel;
};

struct Ep {
    OrtEp base;                     // first member
    Factory* factory = nullptr;
    const OrtApi* api = nullptr;
    const OrtEpApi* ep_api = nullptr;
    int device = 0;
    mnb_session* session = nullptr;
    bool keep_constant_initializers = false;
    bool claim_enabled = true;
    bool qmoe_unfused_as_interleaved = false;   // ep.qmoe_unfused_as_interleaved
    bool strip_major_weights = true;            // ep.strip_major_weights: mnb_weights_prepack
    // Device-memory mode: the HBM memory device ORT places this EP's tensors on (owned by the
    // factory's memory info), else null.
    const OrtMemoryDevice* memory_device = nullptr;
    std::mutex mu;
};

struct Factory {
    OrtEpFactory base;              // first member
    const OrtApi* api = nullptr;
    const OrtEpApi* ep_api = nullptr;
    uint32_t version = 0;
    std::string registered_name;
    bool device_memory = false;     // MI355X_EP_DEVICE_MEMORY, read once at CreateEpFactories
    std::mutex mi_mu;
    std::map<int, OrtMemoryInfo*> memory_infos;   // per HIP device; released with the factory
};

// The OrtMemoryInfo describing HIP device `device`'s HBM, created once and owned by the factory
// (ORT keeps pointers to what EpDevice_AddAllocatorInfo registers).
const OrtMemoryInfo* factory_memory_info(Factory* f, int device) {
    std::lock_guard<std::mutex> lk(f->mi_mu);
    auto it = f->memory_infos.find(device);
    if (it != f->memory_infos.end()) return it->second;
    const std::string name = "MI355X_HBM_" + std::to_string(device);
    OrtMemoryInfo* mi = nullptr;
    ort_check(f->api,
              f->api->CreateMemoryInfo_V2(name.c_str(), OrtMemoryInfoDeviceType_GPU, kAmdVendorId,
                                          device, OrtDeviceMemoryType_DEFAULT, 256,
                                          OrtDeviceAllocator, &mi),
              "CreateMemoryInfo_V2");
    f->memory_infos[device] = mi;
    return mi;
}

// Whether an ORT memory device is this EP's HBM (an AMD GPU's default memory), and which HIP
// ordinal it names.
bool is_our_hbm(const OrtEpApi* ep_api, const OrtMemoryDevice* md, int* device) {
    if (!md) return false;
    if (ep_api->MemoryDevice_GetDeviceType(md) != OrtMemoryInfoDeviceType_GPU) return false;
    if (ep_api->MemoryDevice_GetVendorId(md) != kAmdVendorId) return false;
    if (ep_api->MemoryDevice_GetMemoryType(md) != OrtDeviceMemoryType_DEFAULT) return false;
    if (device) *device = (int)ep_api->MemoryDevice_GetDeviceId(md);
    return true;
}

Factory* as_factory(const OrtEpFactory* p) {
    return reinterpret_cast<Factory*>(const_cast<OrtEpFactory*>(p));
}
Ep* as_ep(const OrtEp* p) { return reinterpret_cast<Ep*>(const_cast<OrtEp*>(p)); }
ComputeInfo* as_info(OrtNodeComputeInfo* p) { return reinterpret_cast<ComputeInfo*>(p); }

// ---- OrtNodeComputeInfo -------------------------------------------------------------------------

OrtStatus* ORT_API_CALL ci_create_state(OrtNodeComputeInfo* self, OrtNodeComputeContext*,
                                        void** state) noexcept {
    if (state) *state = self;
    return nullptr;
}

void ORT_API_CALL ci_release_state(OrtNodeComputeInfo*, void*) noexcept {}

const void* tensor_data(const OrtApi* api, const OrtValue* v) {
    const void* p = nullptr;
    ORT_OK(api, GetTensorData(v, &p));
    return p;
}

size_t tensor_bytes(const OrtApi* api, const OrtValue* v) {
    size_t n = 0;
    ORT_OK(api, GetTensorSizeInBytes(v, &n));
    return n;
}

int32_t tensor_elem_type(const OrtApi* api, const OrtValue* v, std::vector<int64_t>* dims) {
    OrtTensorTypeAndShapeInfo* info = nullptr;
    ORT_OK(api, GetTensorTypeAndShape(v, &info));
    ONNXTensorElementDataType et = ONNX_TENSOR_ELEMENT_DATA_TYPE_UNDEFINED;
    size_t rank = 0;
    OrtStatus* st = api->GetTensorElementType(info, &et);
    if (!st) st = api->GetDimensionsCount(info, &rank);
    if (!st && dims) {
        dims->assign(rank, 0);
        if (rank) st = api->GetDimensions(info, dims->data(), rank);
    }
    api->ReleaseTensorTypeAndShapeInfo(info);
    ort_check(api, st, "reading a tensor's type and shape");
    return (int32_t)et;
}

// ---- streams (device-memory mode) -------------------------------------------------------------
// ORT's stream-aware EP contract (onnxruntime_ep_c_api.h: OrtEpFactory::IsStreamAware and
// CreateSyncStreamForDevice, OrtSyncStreamImpl, OrtSyncNotificationImpl).  Each ORT stream on an
// MI355X device is an async mnb_session of its own -- a hipStream_t with its own staging buffers
// and workspace -- so Compute calls on different ORT streams share no buffer.  Compute enqueues
// on the stream of its kernel context and returns without waiting when its tensors are in HBM;
// ORT orders streams through notifications (hipEvents) and the run's end synchronises.  The
// reference declines streams (rust/src/factory.rs:1268-1280: IsStreamAware false,
// CreateSyncStreamForDevice null), so every one of its Computes waits for the GPU.
struct SyncStream {
    OrtSyncStreamImpl base;         // first member
    Factory* factory = nullptr;
    int device = 0;
    mnb_session* session = nullptr;
};

struct SyncNote {
    OrtSyncNotificationImpl base;   // first member
    SyncStream* producer = nullptr;
    void* event = nullptr;          // hipEvent_t
};

std::mutex g_stream_mu;
std::map<void*, SyncStream*> g_streams;   // hipStream_t of each live SyncStream

SyncStream* stream_of_handle(void* h) {
    if (!h) return nullptr;
    std::lock_guard<std::mutex> lk(g_stream_mu);
    auto it = g_streams.find(h);
    return it == g_streams.end() ? nullptr : it->second;
}

bool any_streams() {
    std::lock_guard<std::mutex> lk(g_stream_mu);
    return !g_streams.empty();
}

// The hipStream_t behind an ORT stream, when it is one of this EP's, else null.
void* our_stream_handle(const OrtApi* api, OrtSyncStream* st) {
    if (!st || !api->SyncStream_GetHandle) return nullptr;
    void* h = api->SyncStream_GetHandle(st);
    return stream_of_handle(h) ? h : nullptr;
}

// The session a Compute runs on: the async session of the ORT stream in its kernel context
// (stream-aware mode), else the EP's own synchronous session.
mnb_session* compute_session(Ep* ep, OrtKernelContext* ctx) {
    if (ep->memory_device && ep->api->KernelContext_GetGPUComputeStream) {
        void* h = nullptr;
        OrtStatus* st = ep->api->KernelContext_GetGPUComputeStream(ctx, &h);
        if (st) {
            ep->api->ReleaseStatus(st);
            h = nullptr;
        }
        SyncStream* ss = stream_of_handle(h);
        if (ss && ss->device == ep->device) return ss->session;
    }
    return ep->session;
}

// Whether a tensor lives in this EP's HBM (device-memory mode), checking the device ordinal.
bool on_our_device(Ep* ep, const OrtValue* v) {
    if (!ep->memory_device || !v) return false;
    int d = -1;
    if (!is_our_hbm(ep->ep_api, ep->ep_api->Value_GetMemoryDevice(v), &d)) return false;
    if (d != ep->device)
        fail(ORT_INVALID_ARGUMENT, "a tensor lives on HIP device %d, this EP runs on %d", d, ep->device);
    return true;
}

void compute_qmoe(Ep* ep, NodeKernel& k, OrtKernelContext* ctx) {
    const OrtApi* api = ep->api;
    size_t nin = 0;
    ORT_OK(api, KernelContext_GetInputCount(ctx, &nin));
    if (k.fused_a >= nin || k.fused_router >= nin)
        fail(ORT_EP_FAIL, "fused QMoE node has %zu inputs", nin);
    const OrtValue* x = nullptr;
    const OrtValue* r = nullptr;
    ORT_OK(api, KernelContext_GetInput(ctx, k.fused_a, &x));
    ORT_OK(api, KernelContext_GetInput(ctx, k.fused_router, &r));
    if (!x || !r) fail(ORT_INVALID_ARGUMENT, "input or router_probs is missing");
    std::vector<int64_t> xd, rd;
    if (tensor_elem_type(api, x, &xd) != kElemFloat16)
        fail(ORT_INVALID_ARGUMENT, "QMoE input is not float16");
    if (tensor_elem_type(api, r, &rd) != k.router_elem)
        fail(ORT_INVALID_ARGUMENT, "router_probs has another element type than at Compile");
    if (xd.empty() || xd.back() != k.qprob.hidden)
        fail(ORT_INVALID_ARGUMENT, "input's last dimension is not the hidden size %lld",
             (long long)k.qprob.hidden);
    int64_t rows = 1;
    for (size_t i = 0; i + 1 < xd.size(); ++i) {
        if (xd[i] < 0) fail(ORT_INVALID_ARGUMENT, "input has a negative extent");
        rows *= xd[i];
    }
    if (rd.size() != 2 || rd[0] != rows || rd[1] != k.qprob.num_experts)
        fail(ORT_INVALID_ARGUMENT, "router_probs must be [%lld, %lld]", (long long)rows,
             (long long)k.qprob.num_experts);
    OrtValue* y = nullptr;
    ORT_OK(api, KernelContext_GetOutput(ctx, 0, xd.data(), xd.size(), &y));
    if (!y) fail(ORT_EP_FAIL, "ORT returned no output tensor");
    if (rows == 0) return;
    void* ydata = nullptr;
    ORT_OK(api, GetTensorMutableData(y, &ydata));
    const bool x_dev = on_our_device(ep, x), r_dev = on_our_device(ep, r), y_dev = on_our_device(ep, y);
    std::lock_guard<std::mutex> lk(k.mu);
    mnb_ok(mnb_session_run_qmoe(compute_session(ep, ctx), k.qweights, rows, tensor_data(api, x), x_dev ? 1 : 0,
                                tensor_data(api, r), r_dev ? 1 : 0, ydata, y_dev ? 1 : 0),
           "QMoE kernels");
    g_compute_count.fetch_add(1);
}

void compute_norm(Ep* ep, NodeKernel& k, OrtKernelContext* ctx) {
    const OrtApi* api = ep->api;
    size_t nin = 0;
    ORT_OK(api, KernelContext_GetInputCount(ctx, &nin));
    if (k.fused_a >= nin || (k.nprob.has_skip && k.fused_skip >= nin))
        fail(ORT_EP_FAIL, "fused norm node has %zu inputs", nin);
    const OrtValue* x = nullptr;
    const OrtValue* sk = nullptr;
    ORT_OK(api, KernelContext_GetInput(ctx, k.fused_a, &x));
    if (k.nprob.has_skip) ORT_OK(api, KernelContext_GetInput(ctx, k.fused_skip, &sk));
    if (!x || (k.nprob.has_skip && !sk)) fail(ORT_INVALID_ARGUMENT, "the input or skip is missing");
    const int32_t want = k.nprob.dtype == MNB_DTYPE_F16 ? kElemFloat16 : kElemFloat;
    std::vector<int64_t> xd, kd;
    if (tensor_elem_type(api, x, &xd) != want) fail(ORT_INVALID_ARGUMENT, "input element type changed");
    if (xd.empty() || xd.back() != k.nprob.hidden)
        fail(ORT_INVALID_ARGUMENT, "input's last dimension is not %lld", (long long)k.nprob.hidden);
    int64_t rows = 1;
    for (size_t i = 0; i + 1 < xd.size(); ++i) {
        if (xd[i] < 0) fail(ORT_INVALID_ARGUMENT, "input has a negative extent");
        rows *= xd[i];
    }
    if (sk && (tensor_elem_type(api, sk, &kd) != want || kd != xd))
        fail(ORT_INVALID_ARGUMENT, "skip's type or shape differs from the input's");
    OrtValue* y = nullptr;
    OrtValue* sum = nullptr;
    ORT_OK(api, KernelContext_GetOutput(ctx, k.fused_y, xd.data(), xd.size(), &y));
    if (k.fused_sum != SIZE_MAX)
        ORT_OK(api, KernelContext_GetOutput(ctx, k.fused_sum, xd.data(), xd.size(), &sum));
    if (!y || (k.fused_sum != SIZE_MAX && !sum)) fail(ORT_EP_FAIL, "ORT returned no output tensor");
    if (rows == 0) return;
    void* yd = nullptr;
    void* sd = nullptr;
    ORT_OK(api, GetTensorMutableData(y, &yd));
    if (sum) ORT_OK(api, GetTensorMutableData(sum, &sd));
    std::lock_guard<std::mutex> lk(k.mu);
    mnb_ok(mnb_session_run_rmsnorm(compute_session(ep, ctx), k.nweights, rows, tensor_data(api, x),
                                   on_our_device(ep, x) ? 1 : 0, sk ? tensor_data(api, sk) : nullptr,
                                   on_our_device(ep, sk) ? 1 : 0, yd, on_our_device(ep, y) ? 1 : 0,
                                   sd, on_our_device(ep, sum) ? 1 : 0),
           "RMSNorm kernel");
    g_compute_count.fetch_add(1);
}

// One GroupQueryAttention Compute.  present's length is the declared one when the graph states
// it (shared buffer or growing), else past + S (growing), as translate_gqa decides
// (rust/src/ops/attention.rs:585-600).
void compute_gqa(Ep* ep, NodeKernel& k, OrtKernelContext* ctx) {
    const OrtApi* api = ep->api;
    size_t nin = 0;
    ORT_OK(api, KernelContext_GetInputCount(ctx, &nin));
    const OrtValue* in[6] = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    for (int i = 0; i < 6; ++i) {
        if (k.gqa_in[i] == SIZE_MAX) continue;
        if (k.gqa_in[i] >= nin) fail(ORT_EP_FAIL, "fused GroupQueryAttention node has %zu inputs", nin);
        ORT_OK(api, KernelContext_GetInput(ctx, k.gqa_in[i], &in[i]));
        if (!in[i]) fail(ORT_INVALID_ARGUMENT, "GroupQueryAttention input %d is missing", i);
    }
    const mnb_gqa_problem& n = k.gprob;
    std::vector<int64_t> qd, pkd, pvd, sd, cd, snd;
    if (tensor_elem_type(api, in[0], &qd) != kElemFloat16 || qd.size() != 3 || qd[2] != k.gqa_packed)
        fail(ORT_INVALID_ARGUMENT, "packed_qkv must be float16 [B, S, %lld]", (long long)k.gqa_packed);
    const int64_t B = qd[0], S = qd[1];
    if (B < 0 || S < 0) fail(ORT_INVALID_ARGUMENT, "packed_qkv has a negative extent");
    if (tensor_elem_type(api, in[1], &pkd) != kElemFloat16 ||
        tensor_elem_type(api, in[2], &pvd) != kElemFloat16 || pkd.size() != 4 || pkd != pvd ||
        pkd[0] != B || pkd[1] != n.kv_num_heads || pkd[3] != n.head_dim || pkd[2] < 0)
        fail(ORT_INVALID_ARGUMENT, "past_key/past_value must be float16 [%lld, %d, L, %d]",
             (long long)B, n.kv_num_heads, n.head_dim);
    if (tensor_elem_type(api, in[3], &sd) != kElemInt32 || sd.size() != 1 || sd[0] != B)
        fail(ORT_INVALID_ARGUMENT, "seqlens_k must be int32 [%lld]", (long long)B);
    int64_t max_seq = n.max_seq;
    if (in[4]) {
        if (tensor_elem_type(api, in[4], &cd) != kElemFloat16 ||
            tensor_elem_type(api, in[5], &snd) != kElemFloat16 || cd.size() != 2 || cd != snd ||
            cd[1] != n.rotary_dim / 2 || cd[0] < 1)
            fail(ORT_INVALID_ARGUMENT, "cos_cache/sin_cache must be float16 [max_seq, %d]",
                 n.rotary_dim / 2);
        max_seq = cd[0];
    }
    mnb_gqa_problem p = n;
    p.batch = B;
    p.seq_len = S;
    p.past_len_max = pkd[2];
    p.present_len = k.gqa_present_len > 0 ? k.gqa_present_len : pkd[2] + S;
    p.max_seq = max_seq;
    mnb_ok(mnb_gqa_check(&p), "GroupQueryAttention shapes");
    const int64_t od[3] = {B, S, (int64_t)n.num_heads * n.head_dim};
    const int64_t kd[4] = {B, n.kv_num_heads, p.present_len, n.head_dim};
    OrtValue* out[3] = {nullptr, nullptr, nullptr};
    ORT_OK(api, KernelContext_GetOutput(ctx, k.gqa_out[0], od, 3, &out[0]));
    ORT_OK(api, KernelContext_GetOutput(ctx, k.gqa_out[1], kd, 4, &out[1]));
    ORT_OK(api, KernelContext_GetOutput(ctx, k.gqa_out[2], kd, 4, &out[2]));
    if (!out[0] || !out[1] || !out[2]) fail(ORT_EP_FAIL, "ORT returned no output tensor");
    if (B == 0 || S == 0) return;
    void* o[3] = {nullptr, nullptr, nullptr};
    for (int i = 0; i < 3; ++i) ORT_OK(api, GetTensorMutableData(out[i], &o[i]));
    const bool past_dev = on_our_device(ep, in[1]);
    if (past_dev != on_our_device(ep, in[2]))
        fail(ORT_INVALID_ARGUMENT, "past_key and past_value live in different memories");
    const bool pres_dev = on_our_device(ep, out[1]);
    if (pres_dev != on_our_device(ep, out[2]))
        fail(ORT_INVALID_ARGUMENT, "present_key and present_value live in different memories");
    uint32_t flags = 0;
    if (on_our_device(ep, in[0])) flags |= MNB_GQA_ON_DEVICE_QKV;
    if (past_dev) flags |= MNB_GQA_ON_DEVICE_PAST;
    if (on_our_device(ep, in[3])) flags |= MNB_GQA_ON_DEVICE_SEQLENS;
    if (on_our_device(ep, out[0])) flags |= MNB_GQA_ON_DEVICE_OUT;
    if (pres_dev) flags |= MNB_GQA_ON_DEVICE_PRESENT;
    if (in[4]) {
        if (on_our_device(ep, in[4]) != on_our_device(ep, in[5]))
            fail(ORT_INVALID_ARGUMENT, "cos_cache and sin_cache live in different memories");
        if (on_our_device(ep, in[4])) flags |= MNB_GQA_ON_DEVICE_CACHES;
    }
    std::lock_guard<std::mutex> lk(k.mu);
    mnb_ok(mnb_session_run_gqa(compute_session(ep, ctx), k.gcaches, &p, tensor_data(api, in[0]),
                               tensor_data(api, in[1]), tensor_data(api, in[2]),
                               static_cast<const int32_t*>(tensor_data(api, in[3])),
                               in[4] ? tensor_data(api, in[4]) : nullptr,
                               in[5] ? tensor_data(api, in[5]) : nullptr, o[0], o[1], o[2], flags),
           "GroupQueryAttention kernels");
    g_compute_count.fetch_add(1);
}

void compute_node(Ep* ep, NodeKernel& k, OrtKernelContext* ctx) {
    const OrtApi* api = ep->api;
    if (env_flag("MI355X_EP_FORCE_COMPUTE_FAILURE"))
        fail(ORT_EP_FAIL, "forced Compute failure (MI355X_EP_FORCE_COMPUTE_FAILURE is set)");
    if (k.qmoe) {
        compute_qmoe(ep, k, ctx);
        return;
    }
    if (k.norm) {
        compute_norm(ep, k, ctx);
        return;
    }
    if (k.gqa) {
        compute_gqa(ep, k, ctx);
        return;
    }
    size_t nin = 0;
    ORT_OK(api, KernelContext_GetInputCount(ctx, &nin));
    if (k.fused_a >= nin) fail(ORT_EP_FAIL, "fused node has %zu inputs; A expected at %zu", nin, k.fused_a);
    const OrtValue* a = nullptr;
    ORT_OK(api, KernelContext_GetInput(ctx, k.fused_a, &a));
    if (!a) fail(ORT_INVALID_ARGUMENT, "input A is missing");
    std::vector<int64_t> adims;
    const int32_t at = tensor_elem_type(api, a, &adims);
    const int32_t want = k.prob.dtype == MNB_DTYPE_F16 ? kElemFloat16 : kElemFloat;
    if (at != want) fail(ORT_INVALID_ARGUMENT, "A has element type %d, the node was compiled for %d", at, want);
    if (adims.empty() || adims.back() != k.prob.k)
        fail(ORT_INVALID_ARGUMENT, "A's last dimension is not K = %lld", (long long)k.prob.k);
    int64_t m = 1;
    for (size_t i = 0; i + 1 < adims.size(); ++i) {
        if (adims[i] < 0) fail(ORT_INVALID_ARGUMENT, "A has a negative extent");
        m *= adims[i];
    }
    std::vector<int64_t> ydims(adims.begin(), adims.end() - 1);
    ydims.push_back(k.prob.n);
    OrtValue* y = nullptr;
    ORT_OK(api, KernelContext_GetOutput(ctx, 0, ydims.data(), ydims.size(), &y));
    if (!y) fail(ORT_EP_FAIL, "ORT returned no output tensor");
    if (m == 0) return;
    void* ydata = nullptr;
    ORT_OK(api, GetTensorMutableData(y, &ydata));
    const void* adata = tensor_data(api, a);

    // Where A and Y live: host memory, or (device-memory mode) this EP's HBM.
    bool a_dev = false, y_dev = false;
    if (ep->memory_device) {
        int da = -1, dy = -1;
        a_dev = is_our_hbm(ep->ep_api, ep->ep_api->Value_GetMemoryDevice(a), &da);
        y_dev = is_our_hbm(ep->ep_api, ep->ep_api->Value_GetMemoryDevice(y), &dy);
        if ((a_dev && da != ep->device) || (y_dev && dy != ep->device))
            fail(ORT_INVALID_ARGUMENT, "a tensor lives on HIP device %d, this EP runs on %d",
                 a_dev && da != ep->device ? da : dy, ep->device);
    }

    std::lock_guard<std::mutex> lk(k.mu);
    mnb_session* sess = compute_session(ep, ctx);
    if (!k.resident) {
        // Weights that are not constant initializers arrive with every call: upload them.  The
        // stream first finishes what it has enqueued (an earlier node may write a weight input,
        // and the previous upload may still be read).
        if (sess != ep->session) mnb_ok(mnb_session_synchronize(sess), "draining the stream");
        const void* host[3] = {nullptr, nullptr, nullptr};
        size_t bytes[3] = {0, 0, 0};
        std::vector<uint8_t> staged[3];
        for (int r = 0; r < 3; ++r) {
            if (k.fused_w[r] == SIZE_MAX) continue;
            if (k.fused_w[r] >= nin) fail(ORT_EP_FAIL, "weight input %d is missing", r + 1);
            const OrtValue* v = nullptr;
            ORT_OK(api, KernelContext_GetInput(ctx, k.fused_w[r], &v));
            if (!v) continue;
            host[r] = tensor_data(api, v);
            bytes[r] = tensor_bytes(api, v);
            int dw = -1;
            if (ep->memory_device && is_our_hbm(ep->ep_api, ep->ep_api->Value_GetMemoryDevice(v), &dw)) {
                // a weight that ORT placed in HBM: bring it to the host for the upload
                staged[r].resize(bytes[r]);
                mnb_ok(mnb_memcpy(dw, staged[r].data(), host[r], bytes[r], MNB_COPY_DEVICE_TO_HOST),
                       "reading a device-resident weight");
                host[r] = staged[r].data();
            }
        }
        if (k.weights) {
            mnb_weights_release(k.weights);
            k.weights = nullptr;
        }
        mnb_ok(mnb_weights_upload(ep->session, &k.prob, host[0], bytes[0], host[1], bytes[1],
                                  host[2], bytes[2], &k.weights),
               "uploading MatMulNBits weights");
        if (ep->strip_major_weights) prepack_weights(k.weights);
    }
    mnb_ok(mnb_session_run(sess, k.weights, m, adata, a_dev ? 1 : 0, ydata, y_dev ? 1 : 0),
           "MatMulNBits kernel");
    g_compute_count.fetch_add(1);
}

OrtStatus* ORT_API_CALL ci_compute(OrtNodeComputeInfo* self, void*, OrtKernelContext* ctx) noexcept {
    ComputeInfo* ci = as_info(self);
    const OrtApi* api = ci && ci->ep ? ci->ep->api : nullptr;
    return guarded(api, "Compute", [&] {
        if (!ci || !ci->kernel || !ctx) fail(ORT_INVALID_ARGUMENT, "null compute arguments");
        compute_node(ci->ep, *ci->kernel, ctx);
    });
}

// ---- OrtEp ----------------------------------------------------------------------------------

const char* ORT_API_CALL ep_get_name(const OrtEp*) noexcept { return kEpName; }

// Device-memory mode: the HBM of the EP's device (reference: rust/src/ep.rs:423-434, which
// returns null there because its tensors stay in host memory).
OrtStatus* ORT_API_CALL ep_get_default_memory_device(const OrtEp* self,
                                                     const OrtMemoryDevice** device) noexcept {
    if (device) *device = self ? as_ep(self)->memory_device : nullptr;
    return nullptr;
}

// Whether the HIP library implements accuracy_level = 4 (int8 activations) for this node's
// form: asked of its planner, so the claim never runs ahead of the kernels.
bool int8_path_available(const NodeFacts& f) {
    if (!f.has_k || !f.has_n || !f.has_bits || !f.has_block_size) return false;
    mnb_problem p{};
    p.m = 1;
    p.n = f.n;
    p.k = f.k;
    p.bits = (int32_t)f.bits;
    p.block_size = (int32_t)f.block_size;
    p.dtype = !f.inputs.empty() && f.inputs[0].elem_type == kElemFloat16 ? MNB_DTYPE_F16
                                                                         : MNB_DTYPE_F32;
    p.has_zero_points = f.inputs.size() > 3 && f.inputs[3].present;
    p.accuracy_level = 4;
    mnb_plan_info info;
    return mnb_plan(&p, &info) == MNB_OK;
}

void get_capability(Ep* ep, const OrtGraph* graph, OrtEpGraphSupportInfo* support) {
    const OrtApi* api = ep->api;
    size_t n = 0;
    ORT_OK(api, Graph_GetNumNodes(graph, &n));
    std::vector<const OrtNode*> nodes(n, nullptr);
    if (n) ORT_OK(api, Graph_GetNodes(graph, nodes.data(), n));
    // Nodes inside control-flow bodies are declined (reference: rust/src/ep.rs:650-664).
    const OrtNode* parent = nullptr;
    ORT_OK(api, Graph_GetParentNode(graph, &parent));
    if (parent) {
        claim_log("declining %zu node(s) of a nested subgraph", n);
        return;
    }
    if (!ep->claim_enabled) return;
    for (const OrtNode* node : nodes) {
        if (!node) continue;
        const std::string op = node_string(api, node, api->Node_GetOperatorType);
        const std::string dom = node_string(api, node, api->Node_GetDomain);
        if (is_skip_norm(op, dom) || is_plain_norm(op, dom)) {
            const std::string name = node_string(api, node, api->Node_GetName);
            const ClaimDecision d = claim_norm(norm_facts(api, node));
            if (!d.claim) {
                claim_log("decline %s: %s", name.c_str(), d.reason.c_str());
                continue;
            }
            OrtNodeFusionOptions opts{};
            opts.ort_version_supported = ep->factory->version;
            opts.drop_constant_initializers = !ep->keep_constant_initializers;
            ort_check(api, ep->ep_api->EpGraphSupportInfo_AddNodesToFuse(support, &node, 1, &opts),
                      "EpGraphSupportInfo_AddNodesToFuse");
            claim_log("claim %s (%s)", name.c_str(), op.c_str());
            continue;
        }
        if (is_gqa(op, dom)) {
            const std::string name = node_string(api, node, api->Node_GetName);
            const ClaimDecision d = claim_gqa(gqa_facts(api, node));
            if (!d.claim) {
                claim_log("decline %s: %s", name.c_str(), d.reason.c_str());
                continue;
            }
            OrtNodeFusionOptions opts{};
            opts.ort_version_supported = ep->factory->version;
            opts.drop_constant_initializers = !ep->keep_constant_initializers;
            ort_check(api, ep->ep_api->EpGraphSupportInfo_AddNodesToFuse(support, &node, 1, &opts),
                      "EpGraphSupportInfo_AddNodesToFuse");
            claim_log("claim %s (GroupQueryAttention)", name.c_str());
            continue;
        }
        if (is_qmoe(op, dom)) {
            const std::string name = node_string(api, node, api->Node_GetName);
            QmoeFacts qf = qmoe_facts(api, node);
            qf.unfused_as_interleaved = ep->qmoe_unfused_as_interleaved;
            const ClaimDecision d = claim_qmoe(qf);
            if (!d.claim) {
                claim_log("decline %s: %s", name.c_str(), d.reason.c_str());
                continue;
            }
            OrtNodeFusionOptions opts{};
            opts.ort_version_supported = ep->factory->version;
            opts.drop_constant_initializers = !ep->keep_constant_initializers;
            ort_check(api, ep->ep_api->EpGraphSupportInfo_AddNodesToFuse(support, &node, 1, &opts),
                      "EpGraphSupportInfo_AddNodesToFuse");
            claim_log("claim %s (QMoE)", name.c_str());
            continue;
        }
        const NodeFacts f = node_facts(api, node);
        if (!is_matmul_nbits(f)) continue;
        const std::string name = node_string(api, node, api->Node_GetName);
        const ClaimDecision d = claim_matmul_nbits(f, int8_path_available(f));
        if (!d.claim) {
            claim_log("decline %s: %s", name.c_str(), d.reason.c_str());
            continue;
        }
        bool all_const = true;
        for (size_t i = 1; i <= 3 && i < f.inputs.size(); ++i)
            if (f.inputs[i].present && !f.inputs[i].constant) all_const = false;
        OrtNodeFusionOptions opts{};
        opts.ort_version_supported = ep->factory->version;
        opts.drop_constant_initializers = all_const && !ep->keep_constant_initializers;
        ort_check(api, ep->ep_api->EpGraphSupportInfo_AddNodesToFuse(support, &node, 1, &opts),
                  "EpGraphSupportInfo_AddNodesToFuse");
        claim_log("claim %s (K=%lld N=%lld bits=%lld bs=%lld acc=%lld, weights %s)", name.c_str(),
                  (long long)f.k, (long long)f.n, (long long)f.bits, (long long)f.block_size,
                  (long long)f.accuracy_level, opts.drop_constant_initializers ? "dropped" : "kept");
    }
}

OrtStatus* ORT_API_CALL ep_get_capability(OrtEp* self, const OrtGraph* graph,
                                          OrtEpGraphSupportInfo* support) noexcept {
    Ep* ep = as_ep(self);
    return guarded(ep ? ep->api : nullptr, "GetCapability", [&] {
        if (!ep || !graph || !support) fail(ORT_INVALID_ARGUMENT, "null GetCapability argument");
        get_capability(ep, graph, support);
    });
}

// Opens the EP's HIP session on first use.
mnb_session* ep_session(Ep* ep) {
    std::lock_guard<std::mutex> lk(ep->mu);
    if (!ep->session) mnb_ok(mnb_session_create(ep->device, &ep->session), "opening the HIP device");
    return ep->session;
}

// Fused-node input index of each body-node input, matched by value name (SIZE_MAX if absent).
std::vector<size_t> fused_input_map(const OrtApi* api, const OrtNode* node, const OrtNode* fused) {
    const std::vector<const OrtValueInfo*> body_in = node_inputs(api, node);
    const std::vector<const OrtValueInfo*> fused_in = node_inputs(api, fused);
    std::vector<std::string> fused_names;
    for (const OrtValueInfo* vi : fused_in) fused_names.push_back(value_name(api, vi));
    std::vector<size_t> out(body_in.size(), SIZE_MAX);
    for (size_t i = 0; i < body_in.size(); ++i) {
        if (!body_in[i]) continue;
        const std::string nm = value_name(api, body_in[i]);
        for (size_t j = 0; j < fused_names.size(); ++j)
            if (fused_names[j] == nm) {
                out[i] = j;
                break;
            }
    }
    return out;
}

std::unique_ptr<NodeKernel> compile_qmoe(Ep* ep, const OrtNode* node, const OrtNode* fused) {
    const OrtApi* api = ep->api;
    QmoeFacts f = qmoe_facts(api, node);
    f.unfused_as_interleaved = ep->qmoe_unfused_as_interleaved;
    QmoeShape shape;
    const ClaimDecision d = claim_qmoe(f, &shape);
    if (!d.claim) fail(ORT_EP_FAIL, "compiled node fails the QMoE claim predicate: %s", d.reason.c_str());
    auto k = std::make_unique<NodeKernel>();
    k->qmoe = true;
    k->name = node_string(api, node, api->Node_GetName);
    mnb_qmoe_problem& p = k->qprob;
    p.hidden = shape.hidden;
    p.inter = shape.inter;
    p.num_experts = shape.experts;
    p.k = (int32_t)f.k;
    p.block_size = f.block_size == 0 ? 32 : (int32_t)f.block_size;
    p.swiglu_fusion = shape.swiglu_fusion;
    p.normalize_routing = f.normalize_routing_weights != 0;
    p.activation_alpha = f.activation_alpha;
    p.activation_beta = f.activation_beta;
    p.swiglu_limit = f.swiglu_limit;
    p.has_swiglu_limit = f.has_swiglu_limit ? 1 : 0;
    p.router_dtype = f.inputs[1].elem_type == kElemFloat16 ? MNB_DTYPE_F16 : MNB_DTYPE_F32;
    p.dtype = MNB_DTYPE_F16;
    k->router_elem = f.inputs[1].elem_type;
    mnb_ok(mnb_qmoe_check(&p), "QMoE attributes");
    const std::vector<size_t> map = fused_input_map(api, node, fused);
    k->fused_a = map[0];
    k->fused_router = map[1];
    if (k->fused_a == SIZE_MAX || k->fused_router == SIZE_MAX)
        fail(ORT_EP_FAIL, "input or router_probs is not an input of the fused node");
    // Expert tensors: constant initializers (the claim requires it), read now, uploaded once.
    const std::vector<const OrtValueInfo*> body_in = node_inputs(api, node);
    const void* host[6] = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    size_t bytes[6] = {0, 0, 0, 0, 0, 0};
    for (int r = 0; r < 6; ++r) {
        const size_t bi = (size_t)r + 2;
        if (!f.inputs[bi].present) continue;
        const OrtValue* v = nullptr;
        ORT_OK(api, ValueInfo_GetInitializerValue(body_in[bi], &v));
        if (!v) fail(ORT_EP_FAIL, "QMoE input %zu has no initializer value", bi);
        host[r] = tensor_data(api, v);
        bytes[r] = tensor_bytes(api, v);
    }
    mnb_ok(mnb_qmoe_weights_upload(ep_session(ep), &p, shape.per_channel ? 1 : 0, host[0],
                                   bytes[0], host[1], bytes[1], host[2], bytes[2], host[3],
                                   bytes[3], host[4], bytes[4], host[5], bytes[5], &k->qweights),
           "uploading QMoE expert weights at Compile");
    if (ep->strip_major_weights)
        mnb_ok(mnb_qmoe_weights_prepack(k->qweights, nullptr),
               "strip-major copy of the QMoE expert weights");
    k->resident = true;
    return k;
}

// Fused-node output index of each body-node output, matched by value name (SIZE_MAX if absent).
std::vector<size_t> fused_output_map(const OrtApi* api, const OrtNode* node, const OrtNode* fused) {
    const std::vector<const OrtValueInfo*> body = node_outputs(api, node);
    const std::vector<const OrtValueInfo*> fo = node_outputs(api, fused);
    std::vector<size_t> out(body.size(), SIZE_MAX);
    for (size_t i = 0; i < body.size(); ++i) {
        if (!body[i]) continue;
        const std::string nm = value_name(api, body[i]);
        for (size_t j = 0; j < fo.size(); ++j)
            if (fo[j] && value_name(api, fo[j]) == nm) {
                out[i] = j;
                break;
            }
    }
    return out;
}

std::unique_ptr<NodeKernel> compile_norm(Ep* ep, const OrtNode* node, const OrtNode* fused) {
    const OrtApi* api = ep->api;
    const NormFacts f = norm_facts(api, node);
    int64_t hidden = 0;
    const ClaimDecision d = claim_norm(f, &hidden);
    if (!d.claim) fail(ORT_EP_FAIL, "compiled node fails the norm claim predicate: %s", d.reason.c_str());
    const bool skip = is_skip_norm(f.op_type, f.domain);
    auto k = std::make_unique<NodeKernel>();
    k->norm = true;
    k->name = node_string(api, node, api->Node_GetName);
    mnb_rmsnorm_problem& p = k->nprob;
    p.hidden = hidden;
    p.epsilon = f.epsilon;
    p.has_skip = skip ? 1 : 0;
    p.has_bias = skip && f.inputs.size() > 3 && f.inputs[3].present ? 1 : 0;
    p.dtype = f.inputs[0].elem_type == kElemFloat16 ? MNB_DTYPE_F16 : MNB_DTYPE_F32;
    mnb_ok(mnb_rmsnorm_check(&p), "norm attributes");
    const std::vector<size_t> in_map = fused_input_map(api, node, fused);
    const std::vector<size_t> out_map = fused_output_map(api, node, fused);
    k->fused_a = in_map[0];
    if (skip) k->fused_skip = in_map[1];
    if (k->fused_a == SIZE_MAX || (skip && k->fused_skip == SIZE_MAX))
        fail(ORT_EP_FAIL, "the input or skip tensor is not an input of the fused node");
    k->fused_y = out_map[0];
    if (k->fused_y == SIZE_MAX) fail(ORT_EP_FAIL, "output 0 is not an output of the fused node");
    if (skip && out_map.size() > 3) k->fused_sum = out_map[3];
    const std::vector<const OrtValueInfo*> body_in = node_inputs(api, node);
    const size_t gi = skip ? 2 : 1;
    const OrtValue* gv = nullptr;
    const OrtValue* bv = nullptr;
    ORT_OK(api, ValueInfo_GetInitializerValue(body_in[gi], &gv));
    if (p.has_bias) ORT_OK(api, ValueInfo_GetInitializerValue(body_in[3], &bv));
    if (!gv || (p.has_bias && !bv)) fail(ORT_EP_FAIL, "gamma or bias has no initializer value");
    mnb_ok(mnb_rmsnorm_weights_upload(ep_session(ep), &p, tensor_data(api, gv),
                                      tensor_bytes(api, gv), bv ? tensor_data(api, bv) : nullptr,
                                      bv ? tensor_bytes(api, bv) : 0, &k->nweights),
           "uploading norm constants at Compile");
    k->resident = true;
    return k;
}

std::unique_ptr<NodeKernel> compile_gqa(Ep* ep, const OrtNode* node, const OrtNode* fused) {
    const OrtApi* api = ep->api;
    const GqaFacts f = gqa_facts(api, node);
    GqaShape shape;
    const ClaimDecision d = claim_gqa(f, &shape);
    if (!d.claim)
        fail(ORT_EP_FAIL, "compiled node fails the GroupQueryAttention claim predicate: %s",
             d.reason.c_str());
    auto k = std::make_unique<NodeKernel>();
    k->gqa = true;
    k->name = node_string(api, node, api->Node_GetName);
    mnb_gqa_problem& p = k->gprob;
    p.num_heads = (int32_t)f.num_heads;
    p.kv_num_heads = (int32_t)f.kv_num_heads;
    p.head_dim = (int32_t)shape.head_dim;
    p.rotary_dim = (int32_t)shape.rotary_dim;
    p.scale = shape.scale;
    p.dtype = MNB_DTYPE_F16;
    k->gqa_packed = shape.packed;
    k->gqa_present_len = shape.declared_present_len;
    const std::vector<size_t> in_map = fused_input_map(api, node, fused);
    const std::vector<size_t> out_map = fused_output_map(api, node, fused);
    const size_t body[6] = {0, 3, 4, 5, 7, 8};
    // cos/sin: constant initializers are read now and uploaded once; otherwise fused inputs
    const bool resident = f.inputs[7].constant && f.inputs[8].constant;
    for (int i = 0; i < 6; ++i) {
        if (i >= 4 && resident) continue;
        k->gqa_in[i] = in_map[body[i]];
        if (k->gqa_in[i] == SIZE_MAX)
            fail(ORT_EP_FAIL, "GroupQueryAttention input %zu is not an input of the fused node", body[i]);
    }
    for (int i = 0; i < 3; ++i) {
        k->gqa_out[i] = out_map[i];
        if (k->gqa_out[i] == SIZE_MAX)
            fail(ORT_EP_FAIL, "GroupQueryAttention output %d is not an output of the fused node", i);
    }
    const void* cos_host = nullptr;
    const void* sin_host = nullptr;
    size_t cos_bytes = 0, sin_bytes = 0;
    p.max_seq = 1;
    if (resident) {
        const std::vector<const OrtValueInfo*> body_in = node_inputs(api, node);
        const OrtValue* cv = nullptr;
        const OrtValue* sv = nullptr;
        ORT_OK(api, ValueInfo_GetInitializerValue(body_in[7], &cv));
        ORT_OK(api, ValueInfo_GetInitializerValue(body_in[8], &sv));
        if (!cv || !sv) fail(ORT_EP_FAIL, "cos_cache or sin_cache has no initializer value");
        std::vector<int64_t> cd, sd;
        if (tensor_elem_type(api, cv, &cd) != kElemFloat16 ||
            tensor_elem_type(api, sv, &sd) != kElemFloat16 || cd.size() != 2 || cd != sd ||
            cd[1] != p.rotary_dim / 2 || cd[0] < 1)
            fail(ORT_EP_FAIL, "cos/sin caches are not float16 [max_seq, %d]", p.rotary_dim / 2);
        p.max_seq = cd[0];
        cos_host = tensor_data(api, cv);
        sin_host = tensor_data(api, sv);
        cos_bytes = tensor_bytes(api, cv);
        sin_bytes = tensor_bytes(api, sv);
    }
    mnb_ok(mnb_gqa_check(&p), "GroupQueryAttention attributes");
    mnb_ok(mnb_gqa_caches_upload(ep_session(ep), &p, cos_host, cos_bytes, sin_host, sin_bytes,
                                 &k->gcaches),
           "uploading the cos/sin caches at Compile");
    k->resident = resident;
    return k;
}

std::unique_ptr<NodeKernel> compile_one(Ep* ep, const OrtGraph* graph, const OrtNode* fused) {
    const OrtApi* api = ep->api;
    size_t n = 0;
    ORT_OK(api, Graph_GetNumNodes(graph, &n));
    if (n != 1) fail(ORT_EP_FAIL, "a fused island holds %zu nodes, expected 1", n);
    const OrtNode* node = nullptr;
    ORT_OK(api, Graph_GetNodes(graph, &node, 1));
    const std::string op = node_string(api, node, api->Node_GetOperatorType);
    const std::string dom = node_string(api, node, api->Node_GetDomain);
    if (is_qmoe(op, dom)) return compile_qmoe(ep, node, fused);
    if (is_skip_norm(op, dom) || is_plain_norm(op, dom)) return compile_norm(ep, node, fused);
    if (is_gqa(op, dom)) return compile_gqa(ep, node, fused);
    const NodeFacts f = node_facts(api, node);
    const ClaimDecision d = claim_matmul_nbits(f, int8_path_available(f));
    if (!d.claim) fail(ORT_EP_FAIL, "compiled node fails the claim predicate: %s", d.reason.c_str());

    auto k = std::make_unique<NodeKernel>();
    k->name = node_string(api, node, api->Node_GetName);
    k->prob.n = f.n;
    k->prob.k = f.k;
    k->prob.bits = (int32_t)f.bits;
    k->prob.block_size = (int32_t)f.block_size;
    k->prob.dtype = f.inputs[0].elem_type == kElemFloat16 ? MNB_DTYPE_F16 : MNB_DTYPE_F32;
    k->prob.accuracy_level = f.has_accuracy_level ? (int32_t)f.accuracy_level : 0;
    k->prob.has_zero_points = f.inputs.size() > 3 && f.inputs[3].present;
    mnb_ok(mnb_check_problem(&k->prob), "MatMulNBits attributes");

    // Map the body node's inputs to the fused node's inputs by value name.
    const std::vector<const OrtValueInfo*> body_in = node_inputs(api, node);
    const std::vector<const OrtValueInfo*> fused_in = node_inputs(api, fused);
    std::vector<std::string> fused_names;
    for (const OrtValueInfo* vi : fused_in) fused_names.push_back(value_name(api, vi));
    auto fused_index = [&](size_t body_i) -> size_t {
        if (body_i >= body_in.size() || !body_in[body_i]) return SIZE_MAX;
        const std::string nm = value_name(api, body_in[body_i]);
        for (size_t j = 0; j < fused_names.size(); ++j)
            if (fused_names[j] == nm) return j;
        return SIZE_MAX;
    };
    k->fused_a = fused_index(0);
    if (k->fused_a == SIZE_MAX) fail(ORT_EP_FAIL, "input A is not an input of the fused node");

    // Constant weights are read from the graph now and uploaded once.
    bool all_const = true;
    const void* host[3] = {nullptr, nullptr, nullptr};
    size_t bytes[3] = {0, 0, 0};
    for (int r = 0; r < 3; ++r) {
        const size_t bi = (size_t)r + 1;
        k->fused_w[r] = fused_index(bi);
        if (bi >= f.inputs.size() || !f.inputs[bi].present) continue;
        const OrtValue* v = nullptr;
        if (f.inputs[bi].constant) ORT_OK(api, ValueInfo_GetInitializerValue(body_in[bi], &v));
        if (!v) {
            all_const = false;
            continue;
        }
        host[r] = tensor_data(api, v);
        bytes[r] = tensor_bytes(api, v);
    }
    mnb_session* sess = ep_session(ep);
    if (all_const) {
        mnb_ok(mnb_weights_upload(sess, &k->prob, host[0], bytes[0], host[1], bytes[1],
                                  host[2], bytes[2], &k->weights),
               "uploading MatMulNBits weights at Compile");
        if (ep->strip_major_weights) prepack_weights(k->weights);
        k->resident = true;
    } else {
        for (int r = 0; r < 3; ++r) {
            const size_t bi = (size_t)r + 1;
            if (bi < f.inputs.size() && f.inputs[bi].present && k->fused_w[r] == SIZE_MAX)
                fail(ORT_EP_FAIL, "weight input %d is neither constant nor a fused-node input", r + 1);
        }
    }
    return k;
}

OrtStatus* ORT_API_CALL ep_compile(OrtEp* self, const OrtGraph** graphs, const OrtNode** fused,
                                   size_t count, OrtNodeComputeInfo** infos,
                                   OrtNode** ep_context_nodes) noexcept {
    Ep* ep = as_ep(self);
    // Every out-slot is defined before anything can fail (reference: rust/src/ep.rs:1906-1913).
    for (size_t i = 0; infos && i < count; ++i) infos[i] = nullptr;
    for (size_t i = 0; ep_context_nodes && i < count; ++i) ep_context_nodes[i] = nullptr;
    std::vector<ComputeInfo*> made;
    OrtStatus* st = guarded(ep ? ep->api : nullptr, "Compile", [&] {
        if (!ep || !graphs || !fused || !infos) fail(ORT_INVALID_ARGUMENT, "null Compile argument");
        for (size_t i = 0; i < count; ++i) {
            auto ci = std::make_unique<ComputeInfo>();
            std::memset(&ci->base, 0, sizeof(ci->base));
            ci->base.ort_version_supported = ep->factory->version;
            ci->base.CreateState = ci_create_state;
            ci->base.Compute = ci_compute;
            ci->base.ReleaseState = ci_release_state;
            ci->ep = ep;
            ci->kernel = compile_one(ep, graphs[i], fused[i]);
            made.push_back(ci.release());
        }
    });
    if (st) {
        for (ComputeInfo* ci : made) delete ci;      // the kernel releases its weights
        return st;
    }
    for (size_t i = 0; i < count; ++i) infos[i] = &made[i]->base;
    return nullptr;
}

void ORT_API_CALL ep_release_infos(OrtEp*, OrtNodeComputeInfo** infos, size_t n) noexcept {
    for (size_t i = 0; infos && i < n; ++i) {
        delete as_info(infos[i]);                       // the kernel releases its weights
    }
}

// ---- OrtEpFactory ---------------------------------------------------------------------------

const char* ORT_API_CALL f_get_name(const OrtEpFactory*) noexcept { return kEpName; }
const char* ORT_API_CALL f_get_vendor(const OrtEpFactory*) noexcept { return kEpVendor; }
uint32_t ORT_API_CALL f_get_vendor_id(const OrtEpFactory*) noexcept { return kAmdVendorId; }
const char* ORT_API_CALL f_get_version(const OrtEpFactory*) noexcept { return kEpVersion; }
// Stream-aware in device-memory mode (host I/O has no streams to share).
bool ORT_API_CALL f_is_stream_aware(const OrtEpFactory* self) noexcept {
    const Factory* f = as_factory(self);
    return f && f->device_memory;
}

// HIP devices this library can run on (gfx950), in HIP ordinal order.
std::vector<int> usable_hip_devices() {
    std::vector<int> out;
    int count = 0;
    if (mnb_device_count(&count) != MNB_OK) return out;
    for (int i = 0; i < count; ++i) {
        char arch[64] = {0};
        if (mnb_device_arch(i, arch, sizeof(arch)) != MNB_OK) continue;
        if (std::strncmp(arch, "gfx950", 6) == 0) out.push_back(i);
    }
    return out;
}

void get_supported_devices(Factory* f, const OrtHardwareDevice* const* devices, size_t num,
                           OrtEpDevice** ep_devices, size_t max_ep_devices, size_t* num_out) {
    const OrtApi* api = f->api;
    *num_out = 0;
    const std::vector<int> hip = usable_hip_devices();
    if (hip.empty()) {
        claim_log("no gfx950 device is visible; advertising none (models run on the CPU EP)");
        return;
    }
    if (!ep_devices || max_ep_devices == 0) return;
    // Correlate the k-th AMD GPU hardware device with the k-th gfx950 HIP device; fall back to
    // any GPU-typed device (reference: rust/src/factory.rs:~290-330).
    std::vector<const OrtHardwareDevice*> amd, gpus;
    for (size_t i = 0; devices && i < num; ++i) {
        const OrtHardwareDevice* d = devices[i];
        if (!d || api->HardwareDevice_Type(d) != OrtHardwareDeviceType_GPU) continue;
        gpus.push_back(d);
        if (api->HardwareDevice_VendorId(d) == kAmdVendorId) amd.push_back(d);
    }
    const std::vector<const OrtHardwareDevice*>& pool = amd.empty() ? gpus : amd;
    size_t written = 0;
    for (size_t i = 0; i < hip.size() && i < pool.size() && written < max_ep_devices; ++i) {
        OrtKeyValuePairs* meta = nullptr;
        api->CreateKeyValuePairs(&meta);
        const std::string idx = std::to_string(hip[i]);
        char arch[64] = {0};
        mnb_device_arch(hip[i], arch, sizeof(arch));
        if (meta) {
            api->AddKeyValuePair(meta, kMetaDeviceIndex, idx.c_str());
            api->AddKeyValuePair(meta, "mi355x.arch", arch);
            api->AddKeyValuePair(meta, "mi355x.correlation", amd.empty() ? "device_type" : "vendor_id");
        }
        OrtEpDevice* epd = nullptr;
        OrtStatus* st = f->ep_api->CreateEpDevice(&f->base, pool[i], meta, nullptr, &epd);
        if (meta) api->ReleaseKeyValuePairs(meta);
        ort_check(api, st, "CreateEpDevice");
        if (f->device_memory) {
            // Advertise the device's HBM so ORT asks CreateAllocator for it.  A failure leaves
            // a working host-I/O EP (reference: rust/src/factory.rs:406-417, :605-660).
            OrtStatus* as = f->ep_api->EpDevice_AddAllocatorInfo(epd, factory_memory_info(f, hip[i]));
            if (as) claim_log("EpDevice_AddAllocatorInfo failed: %s", status_text(api, as).c_str());
        }
        ep_devices[written++] = epd;
    }
    *num_out = written;
}

OrtStatus* ORT_API_CALL f_get_supported_devices(OrtEpFactory* self,
                                                const OrtHardwareDevice* const* devices,
                                                size_t num, OrtEpDevice** ep_devices,
                                                size_t max_ep_devices, size_t* num_out) noexcept {
    Factory* f = as_factory(self);
    return guarded(f ? f->api : nullptr, "GetSupportedDevices", [&] {
        if (!f || !num_out) fail(ORT_INVALID_ARGUMENT, "null GetSupportedDevices argument");
        get_supported_devices(f, devices, num, ep_devices, max_ep_devices, num_out);
    });
}

OrtStatus* ORT_API_CALL f_create_ep(OrtEpFactory* self, const OrtHardwareDevice* const*,
                                    const OrtKeyValuePairs* const* metadata, size_t num_devices,
                                    const OrtSessionOptions* so, const OrtLogger*, OrtEp** out) noexcept {
    Factory* f = as_factory(self);
    if (out) *out = nullptr;
    return guarded(f ? f->api : nullptr, "CreateEp", [&] {
        if (!f || !out) fail(ORT_INVALID_ARGUMENT, "null CreateEp argument");
        if (num_devices != 1)
            fail(ORT_INVALID_ARGUMENT, "one device per session is supported, %zu were selected",
                 num_devices);
        const OrtApi* api = f->api;
        int device = -1;
        if (metadata && metadata[0]) {
            const char* v = api->GetKeyValue(metadata[0], kMetaDeviceIndex);
            if (v && *v) device = std::atoi(v);
        }
        std::string opt;
        if (device < 0 && session_option(api, so, "ep.device_index", &opt)) device = std::atoi(opt.c_str());
        if (device < 0) device = 0;
        auto ep = std::make_unique<Ep>();
        std::memset(&ep->base, 0, sizeof(ep->base));
        ep->base.ort_version_supported = f->version;
        ep->base.GetName = ep_get_name;
        ep->base.GetCapability = ep_get_capability;
        ep->base.Compile = ep_compile;
        ep->base.ReleaseNodeComputeInfos = ep_release_infos;
        ep->factory = f;
        ep->api = api;
        ep->ep_api = f->ep_api;
        ep->device = device;
        if (f->device_memory) {
            ep->memory_device = f->ep_api->MemoryInfo_GetMemoryDevice(factory_memory_info(f, device));
            if (f->version >= 27) ep->base.GetDefaultMemoryDevice = ep_get_default_memory_device;
        }
        if (session_option(api, so, "ep.keep_constant_initializers", &opt))
            ep->keep_constant_initializers = opt == "1" || opt == "true";
        if (session_option(api, so, "ep.qmoe_unfused_as_interleaved", &opt))
            ep->qmoe_unfused_as_interleaved = opt == "1" || opt == "true";
        // ep.strip_major_weights (on unless "0" / "false"): each MatMulNBits node the batched
        // decode kernels can run, and each QMoE node, also keeps a copy of its weights in the
        // MFMA-native strip order (twice the node's weight memory: a few GB of the 288 GB)
        if (session_option(api, so, "ep.strip_major_weights", &opt))
            ep->strip_major_weights = !(opt == "0" || opt == "false");
        // ep.max_claim_ops: comma-separated allowlist (reference: rust/src/ep.rs:39-160);
        // claiming is on only when MatMulNBits is listed.
        if (session_option(api, so, "ep.max_claim_ops", &opt))
            ep->claim_enabled = opt.find("MatMulNBits") != std::string::npos;
        // The HIP device is opened by the first Compile, so creating a session (and claiming
        // nodes) costs no device work.
        *out = &ep.release()->base;
    });
}

void ORT_API_CALL f_release_ep(OrtEpFactory*, OrtEp* p) noexcept {
    Ep* ep = as_ep(p);
    if (!ep) return;
    if (ep->session) mnb_session_destroy(ep->session);
    delete ep;
}

// ---- device memory: allocator and data transfer --------------------------------------------

// An OrtAllocator over hipMalloc on one HIP device (reference counterpart: the Vulkan handle
// allocator, rust/src/allocator.rs).  The memory info it reports is the factory's.
struct DeviceAllocator {
    OrtAllocator base;              // first member
    int device = 0;
    const OrtMemoryInfo* info = nullptr;
};

void* ORT_API_CALL da_alloc(OrtAllocator* self, size_t size) noexcept {
    auto* a = reinterpret_cast<DeviceAllocator*>(self);
    void* p = nullptr;
    if (!a || mnb_device_malloc(a->device, size, &p) != MNB_OK) return nullptr;
    return p;
}

void ORT_API_CALL da_free(OrtAllocator* self, void* p) noexcept {
    auto* a = reinterpret_cast<DeviceAllocator*>(self);
    if (a && p) (void)mnb_device_free(a->device, p);
}

const OrtMemoryInfo* ORT_API_CALL da_info(const OrtAllocator* self) noexcept {
    return self ? reinterpret_cast<const DeviceAllocator*>(self)->info : nullptr;
}

OrtStatus* ORT_API_CALL f_create_allocator(OrtEpFactory* self, const OrtMemoryInfo* memory_info,
                                           const OrtKeyValuePairs*, OrtAllocator** out) noexcept {
    if (out) *out = nullptr;        // defined before anything can fail
    Factory* f = as_factory(self);
    return guarded(f ? f->api : nullptr, "CreateAllocator", [&] {
        if (!f || !out || !memory_info || !f->device_memory) return;   // host I/O: no allocator
        int device = -1;
        if (!is_our_hbm(f->ep_api, f->ep_api->MemoryInfo_GetMemoryDevice(memory_info), &device))
            return;                 // a memory info this EP did not advertise: decline
        auto a = std::make_unique<DeviceAllocator>();
        std::memset(&a->base, 0, sizeof(a->base));
        a->base.version = f->version;
        a->base.Alloc = da_alloc;
        a->base.Free = da_free;
        a->base.Info = da_info;
        a->base.Reserve = da_alloc;
        a->device = device;
        a->info = factory_memory_info(f, device);
        *out = &a.release()->base;
    });
}

void ORT_API_CALL f_release_allocator(OrtEpFactory*, OrtAllocator* a) noexcept {
    delete reinterpret_cast<DeviceAllocator*>(a);
}

// Host <-> HBM and HBM <-> HBM copies of whole tensors (reference: rust/src/transfer.rs).
struct DataTransfer {
    OrtDataTransferImpl base;       // first member
    Factory* factory = nullptr;
};

void ORT_API_CALL dt_release(OrtDataTransferImpl* self) noexcept {
    delete reinterpret_cast<DataTransfer*>(self);
}

bool ORT_API_CALL dt_can_copy(const OrtDataTransferImpl* self, const OrtMemoryDevice* src,
                              const OrtMemoryDevice* dst) noexcept {
    const auto* t = reinterpret_cast<const DataTransfer*>(self);
    if (!t || !src || !dst) return false;
    const OrtEpApi* e = t->factory->ep_api;
    const bool s_hbm = is_our_hbm(e, src, nullptr), d_hbm = is_our_hbm(e, dst, nullptr);
    const bool s_host = e->MemoryDevice_GetDeviceType(src) == OrtMemoryInfoDeviceType_CPU;
    const bool d_host = e->MemoryDevice_GetDeviceType(dst) == OrtMemoryInfoDeviceType_CPU;
    return (s_hbm && (d_hbm || d_host)) || (s_host && d_hbm);
}

OrtStatus* ORT_API_CALL dt_copy(OrtDataTransferImpl* self, const OrtValue** src, OrtValue** dst,
                                OrtSyncStream** streams, size_t n) noexcept {
    auto* t = reinterpret_cast<DataTransfer*>(self);
    const OrtApi* api = t ? t->factory->api : nullptr;
    return guarded(api, "CopyTensors", [&] {
        if (!t || (n && (!src || !dst))) fail(ORT_INVALID_ARGUMENT, "null CopyTensors argument");
        const OrtEpApi* e = t->factory->ep_api;
        for (size_t i = 0; i < n; ++i) {
            const size_t sb = tensor_bytes(api, src[i]), db = tensor_bytes(api, dst[i]);
            if (sb != db) fail(ORT_INVALID_ARGUMENT, "copy of %zu bytes into a %zu-byte tensor", sb, db);
            int sd = -1, dd = -1;
            const bool s_hbm = is_our_hbm(e, e->Value_GetMemoryDevice(src[i]), &sd);
            const bool d_hbm = is_our_hbm(e, e->Value_GetMemoryDevice(dst[i]), &dd);
            if (!s_hbm && !d_hbm) fail(ORT_INVALID_ARGUMENT, "neither tensor is in this EP's HBM");
            void* dp = nullptr;
            ORT_OK(api, GetTensorMutableData(dst[i], &dp));
            const void* sp = tensor_data(api, src[i]);
            const int kind = s_hbm && d_hbm ? MNB_COPY_DEVICE_TO_DEVICE
                                            : (s_hbm ? MNB_COPY_DEVICE_TO_HOST : MNB_COPY_HOST_TO_DEVICE);
            const int dev = d_hbm ? dd : sd;
            void* h = our_stream_handle(api, streams ? streams[i] : nullptr);
            if (h) {
                // ordered on the ORT stream: after the kernels that produced the source
                mnb_ok(mnb_memcpy_on_stream(dev, dp, sp, sb, kind, h), "tensor copy");
                continue;
            }
            // no stream: after everything enqueued on this EP's streams (they do not order
            // with the synchronous copy)
            if (any_streams()) mnb_ok(mnb_device_synchronize(dev), "draining the EP's streams");
            mnb_ok(mnb_memcpy(dev, dp, sp, sb, kind), "tensor copy");
        }
    });
}

OrtStatus* ORT_API_CALL f_create_data_transfer(OrtEpFactory* self, OrtDataTransferImpl** out) noexcept {
    if (out) *out = nullptr;
    Factory* f = as_factory(self);
    return guarded(f ? f->api : nullptr, "CreateDataTransfer", [&] {
        if (!f || !out || !f->device_memory) return;     // host I/O needs no copies
        auto t = std::make_unique<DataTransfer>();
        std::memset(&t->base, 0, sizeof(t->base));
        t->base.ort_version_supported = f->version;
        t->base.Release = dt_release;
        t->base.CanCopy = dt_can_copy;
        t->base.CopyTensors = dt_copy;
        t->factory = f;
        *out = &t.release()->base;
    });
}

void ORT_API_CALL sn_release(OrtSyncNotificationImpl* self) noexcept {
    auto* n = reinterpret_cast<SyncNote*>(self);
    if (!n) return;
    (void)mnb_event_destroy(n->event);
    delete n;
}

OrtStatus* ORT_API_CALL sn_activate(OrtSyncNotificationImpl* self) noexcept {
    auto* n = reinterpret_cast<SyncNote*>(self);
    const OrtApi* api = n ? n->producer->factory->api : nullptr;
    return guarded(api, "Notification::Activate", [&] {
        if (!n) fail(ORT_INVALID_ARGUMENT, "null notification");
        mnb_ok(mnb_event_record(n->event, mnb_session_stream(n->producer->session)),
               "recording the notification");
    });
}

OrtStatus* ORT_API_CALL sn_wait_on_device(OrtSyncNotificationImpl* self,
                                          OrtSyncStream* consumer) noexcept {
    auto* n = reinterpret_cast<SyncNote*>(self);
    const OrtApi* api = n ? n->producer->factory->api : nullptr;
    return guarded(api, "Notification::WaitOnDevice", [&] {
        if (!n) fail(ORT_INVALID_ARGUMENT, "null notification");
        void* h = our_stream_handle(api, consumer);
        if (h)
            mnb_ok(mnb_stream_wait_event(h, n->event), "stream wait on the notification");
        else                        // another EP's stream: wait on the host instead
            mnb_ok(mnb_event_synchronize(n->event), "host wait on the notification");
    });
}

OrtStatus* ORT_API_CALL sn_wait_on_host(OrtSyncNotificationImpl* self) noexcept {
    auto* n = reinterpret_cast<SyncNote*>(self);
    const OrtApi* api = n ? n->producer->factory->api : nullptr;
    return guarded(api, "Notification::WaitOnHost", [&] {
        if (!n) fail(ORT_INVALID_ARGUMENT, "null notification");
        mnb_ok(mnb_event_synchronize(n->event), "host wait on the notification");
    });
}

void ORT_API_CALL ss_release(OrtSyncStreamImpl* self) noexcept {
    auto* ss = reinterpret_cast<SyncStream*>(self);
    if (!ss) return;
    {
        std::lock_guard<std::mutex> lk(g_stream_mu);
        g_streams.erase(mnb_session_stream(ss->session));
    }
    (void)mnb_session_destroy(ss->session);      // drains the stream first
    delete ss;
}

void* ORT_API_CALL ss_get_handle(OrtSyncStreamImpl* self) noexcept {
    auto* ss = reinterpret_cast<SyncStream*>(self);
    return ss ? mnb_session_stream(ss->session) : nullptr;
}

OrtStatus* ORT_API_CALL ss_create_notification(OrtSyncStreamImpl* self,
                                               OrtSyncNotificationImpl** out) noexcept {
    if (out) *out = nullptr;
    auto* ss = reinterpret_cast<SyncStream*>(self);
    return guarded(ss ? ss->factory->api : nullptr, "CreateNotification", [&] {
        if (!ss || !out) fail(ORT_INVALID_ARGUMENT, "null CreateNotification argument");
        auto n = std::make_unique<SyncNote>();
        std::memset(&n->base, 0, sizeof(n->base));
        n->base.ort_version_supported = ss->factory->version;
        n->base.Release = sn_release;
        n->base.Activate = sn_activate;
        n->base.WaitOnDevice = sn_wait_on_device;
        n->base.WaitOnHost = sn_wait_on_host;
        n->producer = ss;
        mnb_ok(mnb_event_create(ss->device, &n->event), "creating a notification event");
        *out = &n.release()->base;
    });
}

// HIP streams need no flush: work is submitted as it is enqueued.
OrtStatus* ORT_API_CALL ss_flush(OrtSyncStreamImpl*) noexcept { return nullptr; }

// The end of a run: the stream's work is complete (and its errors reported) before Run returns.
OrtStatus* ORT_API_CALL ss_on_session_run_end(OrtSyncStreamImpl* self) noexcept {
    auto* ss = reinterpret_cast<SyncStream*>(self);
    return guarded(ss ? ss->factory->api : nullptr, "OnSessionRunEnd", [&] {
        if (ss) mnb_ok(mnb_session_synchronize(ss->session), "finishing the run's GPU work");
    });
}

OrtStatus* ORT_API_CALL f_create_sync_stream(OrtEpFactory* self, const OrtMemoryDevice* md,
                                             const OrtKeyValuePairs*, OrtSyncStreamImpl** out) noexcept {
    if (out) *out = nullptr;
    Factory* f = as_factory(self);
    return guarded(f ? f->api : nullptr, "CreateSyncStreamForDevice", [&] {
        if (!f || !out || !f->device_memory) return;     // host I/O: no streams
        int device = -1;
        if (!is_our_hbm(f->ep_api, md, &device)) return; // not this EP's memory: no stream
        auto ss = std::make_unique<SyncStream>();
        std::memset(&ss->base, 0, sizeof(ss->base));
        ss->base.ort_version_supported = f->version;
        ss->base.Release = ss_release;
        ss->base.GetHandle = ss_get_handle;
        ss->base.CreateNotification = ss_create_notification;
        ss->base.Flush = ss_flush;
        ss->base.OnSessionRunEnd = ss_on_session_run_end;
        ss->factory = f;
        ss->device = device;
        mnb_ok(mnb_session_create(device, &ss->session), "opening a HIP stream");
        const int rc = mnb_session_set_async(ss->session, 1);
        if (rc) {
            (void)mnb_session_destroy(ss->session);
            mnb_ok(rc, "async session");
        }
        {
            std::lock_guard<std::mutex> lk(g_stream_mu);
            g_streams[mnb_session_stream(ss->session)] = ss.get();
        }
        *out = &ss.release()->base;
    });
}

// ---- ABI negotiation --------------------------------------------------------------------------

struct Negotiated {
    const OrtApi* api = nullptr;
    const OrtEpApi* ep_api = nullptr;
    uint32_t version = 0;
};

// Asks the host for the newest OrtApi from the built version down to the minimum (reference:
// rust/src/sys.rs:193-277).  Older tables are prefixes of newer ones, and ORT reads our vtables
// only up to the version we report.
Negotiated negotiate(const OrtApiBase* base, std::string* err) {
    Negotiated n;
    if (!base || !base->GetApi) {
        *err = "ONNX Runtime passed no usable OrtApiBase";
        return n;
    }
    for (uint32_t v = kVersionBuilt; v >= kVersionMin; --v) {
        const OrtApi* api = base->GetApi(v);
        if (api) {
            n.api = api;
            n.version = v;
            break;
        }
    }
    if (!n.api) {
        const char* hv = base->GetVersionString ? base->GetVersionString() : nullptr;
        char buf[256];
        std::snprintf(buf, sizeof(buf),
                      "%s requires ONNX Runtime with ORT_API_VERSION >= %u (built against %u); "
                      "this host (%s) offered none of them",
                      kEpName, kVersionMin, kVersionBuilt, hv ? hv : "unknown version");
        *err = buf;
        return n;
    }
    n.ep_api = n.api->GetEpApi ? n.api->GetEpApi() : nullptr;
    if (!n.ep_api) {
        *err = "the host's OrtApi has no OrtEpApi (plugin EPs unsupported)";
        n.api = nullptr;
    }
    return n;
}

}  // namespace
}  // namespace mi355x_ep

using namespace mi355x_ep;

MI355X_EXPORT OrtStatus* CreateEpFactories(const char* registered_name,
                                           const OrtApiBase* ort_api_base, const OrtLogger*,
                                           OrtEpFactory** factories, size_t max_factories,
                                           size_t* num_factories) {
    std::string err;
    const Negotiated n = negotiate(ort_api_base, &err);
    if (!n.api) {
        // Build the error status from the oldest table, whose CreateStatus slot never moved.
        const OrtApi* any = ort_api_base && ort_api_base->GetApi ? ort_api_base->GetApi(1) : nullptr;
        return to_status(any, ORT_INVALID_ARGUMENT, err);
    }
    return guarded(n.api, "CreateEpFactories", [&] {
        if (!factories || !num_factories) fail(ORT_INVALID_ARGUMENT, "null factory out-parameters");
        *num_factories = 0;
        if (max_factories < 1) fail(ORT_INVALID_ARGUMENT, "ORT allowed room for no factory");
        auto f = std::make_unique<Factory>();
        std::memset(&f->base, 0, sizeof(f->base));
        f->api = n.api;
        f->ep_api = n.ep_api;
        f->version = n.version;
        f->registered_name = registered_name ? registered_name : kEpName;
        f->device_memory = device_memory_requested();
        OrtEpFactory& b = f->base;
        b.ort_version_supported = n.version;
        b.GetName = f_get_name;
        b.GetVendor = f_get_vendor;
        b.GetSupportedDevices = f_get_supported_devices;
        b.CreateEp = f_create_ep;
        b.ReleaseEp = f_release_ep;
        b.GetVendorId = f_get_vendor_id;
        b.GetVersion = f_get_version;
        b.CreateAllocator = f_create_allocator;
        b.ReleaseAllocator = f_release_allocator;
        b.CreateDataTransfer = f_create_data_transfer;
        b.IsStreamAware = f_is_stream_aware;
        b.CreateSyncStreamForDevice = f_create_sync_stream;
        factories[0] = &f.release()->base;
        *num_factories = 1;
    });
}

MI355X_EXPORT OrtStatus* ReleaseEpFactory(OrtEpFactory* factory) {
    Factory* f = as_factory(factory);
    if (f) {
        for (auto& kv : f->memory_infos)
            if (kv.second) f->api->ReleaseMemoryInfo(kv.second);
    }
    delete f;
    return nullptr;
}

MI355X_EXPORT uint64_t OrtEpMi355xGetComputeCount(void) { return g_compute_count.load(); }

MI355X_EXPORT void OrtEpMi355xResetComputeCount(void) { g_compute_count.store(0); }
