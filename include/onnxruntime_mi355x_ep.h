/*
 * onnxruntime_mi355x_ep.h — exported C ABI of libonnxruntime_mi355x_ep.so, the ONNX Runtime
 * plugin execution provider that runs com.microsoft::MatMulNBits on an MI355X (gfx950).
 *
 * A stock ONNX Runtime (plugin-EP ABI, ORT_API_VERSION 24..28) loads the library with
 *     ort.register_execution_provider_library("MI355XExecutionProvider", "/path/libonnxruntime_mi355x_ep.so")
 * and resolves exactly the two functions below by name, the same surface the reference plugin
 * exports.  Everything else ORT reaches through the vtables those functions hand back
 * (OrtEpFactory -> OrtEp -> OrtNodeComputeInfo), declared in ORT's own onnxruntime_ep_c_api.h.
 *
 *   CreateEpFactories   replaces rust/src/lib.rs:224-344 (the reference's CreateEpFactories:
 *                       ABI negotiation 28 -> 24, one factory, panic guard -> OrtStatus)
 *   ReleaseEpFactory    replaces rust/src/lib.rs:350-373
 *   OrtEpMi355xGetComputeCount
 *                       diagnostic counter of MatMulNBits Compute calls that launched a kernel,
 *                       the counterpart of OrtEpVulkanGetExecutionCounters
 *                       (rust/src/lib.rs:392); ORT never calls it
 *   OrtEpMi355xResetComputeCount
 *                       counterpart of OrtEpVulkanResetExecutionCounters (rust/src/lib.rs:608)
 *
 * The ORT types are opaque here so that a host can declare the entry points without ORT's
 * headers; their layouts are ORT's (onnxruntime_c_api.h / onnxruntime_ep_c_api.h, v1.28.0).
 */
#ifndef ONNXRUNTIME_MI355X_EP_H_
#define ONNXRUNTIME_MI355X_EP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

struct OrtStatus;
struct OrtApiBase;
struct OrtLogger;
struct OrtEpFactory;

/* Registered EP name the factory reports (OrtEpFactory::GetName / OrtEp::GetName). */
#define MI355X_EP_NAME "MI355XExecutionProvider"

/* ORT plugin-EP ABI versions this library negotiates: built against 28, accepts down to 24. */
#define MI355X_EP_ORT_API_VERSION_BUILT 28
#define MI355X_EP_ORT_API_VERSION_MIN 24

struct OrtStatus* CreateEpFactories(const char* registered_name,
                                    const struct OrtApiBase* ort_api_base,
                                    const struct OrtLogger* default_logger,
                                    struct OrtEpFactory** factories, size_t max_factories,
                                    size_t* num_factories);

struct OrtStatus* ReleaseEpFactory(struct OrtEpFactory* factory);

uint64_t OrtEpMi355xGetComputeCount(void);
void OrtEpMi355xResetComputeCount(void);

#ifdef __cplusplus
}
#endif

#endif /* ONNXRUNTIME_MI355X_EP_H_ */
