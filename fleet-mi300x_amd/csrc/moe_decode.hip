// Launch of the batch-1 MoE layer (the device code is moe_body.h) and its C
// entry points.
#include "moe_body.h"

namespace fleet_moe {
namespace decode {

__global__ __launch_bounds__(kThreads, 1) void moe_decode_kernel(Params P) {
    __shared__ Lds L;
    u32x4 pre[8];
    moe_layer<false>(P, L, pre, false, [] {});
}

}  // namespace decode
}  // namespace fleet_moe

using namespace fleet_moe;

static bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

int fleet_moe_check_dims(const fleet_moe_dims* d);   // moe_abi.hip
int fleet_moe_check_device(int min_cus);              // moe_abi.hip
int fleet_moe_check_resident(const void* fn, int threads, int grid);

#if FLEET_MOE_TRACE
static unsigned long long* g_trace = nullptr;
extern "C" void fleet_moe_debug_set_trace(void* p) { g_trace = (unsigned long long*)p; }
#endif

extern "C" size_t fleet_moe_layer_workspace_bytes(const fleet_moe_dims* dims) {
    (void)dims;
    return (sizeof(decode::Workspace) + 255) & ~(size_t)255;
}

extern "C" int fleet_moe_layer_decode(const fleet_moe_layer* layer, const float* x,
                                      float* x_out, uint16_t* moe_out, int32_t* ids,
                                      float* weights, void* workspace, size_t workspace_bytes,
                                      const fleet_moe_dims* dims, hipStream_t stream) {
    if (!layer || !dims) return FLEET_MOE_ERR_ARG;
    if (int e = fleet_moe_check_dims(dims)) return e;
    if (!layer->router || !layer->experts || !layer->shared || !x || !x_out || !workspace)
        return FLEET_MOE_ERR_ARG;
    if (!aligned(layer->router, 16) || !aligned(layer->experts, 16) ||
        !aligned(layer->shared, 16) || !aligned(x, 16) || !aligned(x_out, 4) ||
        !aligned(workspace, 256) || (layer->norm && !aligned(layer->norm, 8)) ||
        (moe_out && !aligned(moe_out, 2)) || (ids && !aligned(ids, 4)) ||
        (weights && !aligned(weights, 4)))
        return FLEET_MOE_ERR_ARG;
    if (layer->expert_stride < kExpertStride || layer->expert_stride % kChunk != 0)
        return FLEET_MOE_ERR_DIMS;
    if (workspace_bytes < fleet_moe_layer_workspace_bytes(dims)) return FLEET_MOE_ERR_WORKSPACE;
    if (int e = fleet_moe_check_resident(reinterpret_cast<const void*>(&decode::moe_decode_kernel),
                                         decode::kThreads, decode::kWG))
        return e;

    decode::Params P{};
    P.norm = layer->norm;
    P.router = reinterpret_cast<const u32x4*>(layer->router);
    P.experts = layer->experts;
    P.shared = layer->shared;
    P.x = x;
    P.x_out = x_out;
    P.moe_out = moe_out;
    P.ids_out = ids;
    P.w_out = weights;
    P.ws = reinterpret_cast<decode::Workspace*>(workspace);
    P.expert_stride = layer->expert_stride;
    P.eps = dims->rms_eps;
    P.scaling = dims->routed_scaling;
#if FLEET_MOE_TRACE
    P.trace = g_trace;
#endif
    hipLaunchKernelGGL(decode::moe_decode_kernel, dim3(decode::kWG), dim3(decode::kThreads), 0,
                       stream, P);
    return (int)hipGetLastError();
}
