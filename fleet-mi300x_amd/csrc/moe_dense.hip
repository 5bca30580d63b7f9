// Launch of the batch-1 dense SwiGLU layer (the device code is dense_body.h)
// and its C entry points.
#include "dense_body.h"

namespace fleet_moe {
namespace dense {

__global__ __launch_bounds__(kThreads, 1) void dense_kernel(Params P) {
    __shared__ Lds L;
    u32x4 pre[8];
    dense_layer<false>(P, L, pre, false, [] {});
}

}  // namespace dense
}  // namespace fleet_moe

using namespace fleet_moe;

int fleet_moe_check_dims(const fleet_moe_dims* d);
int fleet_moe_check_device(int min_cus);
int fleet_moe_check_resident(const void* fn, int threads, int grid);

static bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

extern "C" size_t fleet_moe_dense_workspace_bytes(const fleet_moe_dims* dims, int32_t dense_inter) {
    if (fleet_moe_check_dims(dims) != 0 || dense_inter != dense::kDenseInter) return 0;
    return (sizeof(dense::Workspace) + 255) & ~(size_t)255;
}

extern "C" int fleet_moe_dense_decode(const uint16_t* norm, const uint16_t* w, int32_t dense_inter,
                                      const float* x, float* x_out, uint16_t* mlp_out,
                                      void* workspace, size_t workspace_bytes,
                                      const fleet_moe_dims* dims, hipStream_t stream) {
    if (int e = fleet_moe_check_dims(dims)) return e;
    if (dense_inter != dense::kDenseInter) return FLEET_MOE_ERR_DIMS;
    if (!w || !x || !x_out || !workspace) return FLEET_MOE_ERR_ARG;
    if (!aligned(w, 16) || !aligned(x, 16) || !aligned(x_out, 16) || !aligned(workspace, 256) ||
        (norm && !aligned(norm, 8)) || (mlp_out && !aligned(mlp_out, 2)))
        return FLEET_MOE_ERR_ARG;
    if (workspace_bytes < sizeof(dense::Workspace)) return FLEET_MOE_ERR_WORKSPACE;
    if (int e = fleet_moe_check_resident(reinterpret_cast<const void*>(&dense::dense_kernel),
                                         dense::kThreads, dense::kWG))
        return e;
    dense::Params P{};
    P.norm = norm;
    P.w = w;
    P.x = x;
    P.x_out = x_out;
    P.mlp_out = mlp_out;
    P.ws = static_cast<dense::Workspace*>(workspace);
    P.eps = dims->rms_eps;
    hipLaunchKernelGGL(dense::dense_kernel, dim3(dense::kWG), dim3(dense::kThreads), 0, stream, P);
    return (int)hipGetLastError();
}
