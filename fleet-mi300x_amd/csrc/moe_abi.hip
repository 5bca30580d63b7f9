// C-ABI plumbing shared by the entry points, and the standalone router.
//
// fleet_moe_router_topk runs the router GEMV and the greedy top-k for any
// number of tokens: one workgroup per token, four waves, 16 router rows per
// wave with fp64 accumulation of the exact bf16 x bf16 products (so the logits
// are the correctly rounded fp32 values and the routing is reproducible bit
// for bit), then softmax + top-k on wave 0 with ties to the lowest index.
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <vector>

#include "moe_common.h"

namespace fleet_moe {

int check_dims_impl(const fleet_moe_dims* d) {
    if (!d) return FLEET_MOE_ERR_ARG;
    if (d->hidden != kHidden || d->moe_inter != kInter || d->n_routed != kRouted ||
        d->n_shared != kShared || d->top_k != kTopK)
        return FLEET_MOE_ERR_DIMS;
    if (!(d->rms_eps > 0.f) || !(d->routed_scaling == d->routed_scaling))
        return FLEET_MOE_ERR_ARG;
    return 0;
}

namespace {
struct DeviceInfo {
    int checked = 0;
    int status = 0;
};
std::mutex g_mu;
std::vector<DeviceInfo> g_dev;
}  // namespace

// Per device, once: the code object is gfx950-only, and the kernels whose
// workgroups wait on each other launch one workgroup per CU over `min_cus` CUs.
int check_device_impl(int min_cus) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    std::lock_guard<std::mutex> lk(g_mu);
    if ((int)g_dev.size() <= dev) g_dev.resize(dev + 1);
    DeviceInfo& di = g_dev[dev];
    if (!di.checked) {
        hipDeviceProp_t prop;
        e = hipGetDeviceProperties(&prop, dev);
        if (e != hipSuccess) return (int)e;
        di.status = (strncmp(prop.gcnArchName, "gfx950", 6) == 0 &&
                     prop.multiProcessorCount >= min_cus)
                        ? 0
                        : FLEET_MOE_ERR_DEVICE;
        di.checked = 1;
    }
    return di.status;
}

namespace {
struct ResidentInfo {
    int dev;
    const void* fn;
    int status;
};
std::vector<ResidentInfo> g_resident;
}  // namespace

// Per device and kernel, once: the kernel's workgroups wait for each other's
// data, so all `grid` of them (one per CU, `threads` threads each) must be
// resident at the same time. That holds when the device has at least `grid`
// CUs and one workgroup fits on a CU with the kernel's registers and LDS;
// otherwise FLEET_MOE_ERR_DEVICE. (Work of other processes or streams holding
// CUs can still delay residency; the kernels' waits are bounded for that.)
int check_resident_impl(const void* fn, int threads, int grid) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return (int)e;
    if (int st = check_device_impl(grid)) return st;
    std::lock_guard<std::mutex> lk(g_mu);
    for (const ResidentInfo& r : g_resident)
        if (r.dev == dev && r.fn == fn) return r.status;
    int per_cu = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, 0);
    if (e != hipSuccess) return (int)e;
    const int st = per_cu >= 1 ? 0 : FLEET_MOE_ERR_DEVICE;
    g_resident.push_back(ResidentInfo{dev, fn, st});
    return st;
}

namespace router {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kLanes;
constexpr int kRowsPerWave = kRouted / kWaves;   // 16

struct Params {
    const u32x4* router;
    const float* x;          // fp32[T][H]
    const float* bias;       // fp32[64] or null
    float* logits;           // fp32[T][64] or null
    int32_t* ids;            // int32[T][6]
    float* weights;          // fp32[T][6]
    float scaling;
};

__global__ __launch_bounds__(kThreads) void router_topk_kernel(Params P) {
    __shared__ float s_logit[kRouted];
    __shared__ int s_ids[8];
    __shared__ float s_w[8];
    const int t = blockIdx.x;
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & (kLanes - 1);
    const float* xt = P.x + (int64_t)t * kHidden;
    float xr[4][8];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        const float4 a = reinterpret_cast<const float4*>(xt)[2 * (lane + kLanes * m)];
        const float4 b = reinterpret_cast<const float4*>(xt)[2 * (lane + kLanes * m) + 1];
        xr[m][0] = a.x; xr[m][1] = a.y; xr[m][2] = a.z; xr[m][3] = a.w;
        xr[m][4] = b.x; xr[m][5] = b.y; xr[m][6] = b.z; xr[m][7] = b.w;
    }
    for (int r = wave * kRowsPerWave; r < (wave + 1) * kRowsPerWave; ++r) {
        const u32x4* row = P.router + (int64_t)r * kRowChunks;
        double acc = 0.0;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const u32x4 w = row[lane + kLanes * m];
            const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc += (double)(bf_lo(wv[q]) * xr[m][2 * q]);
                acc += (double)(bf_hi(wv[q]) * xr[m][2 * q + 1]);
            }
        }
        acc = wave_sum64(acc);
        if (lane == 0) s_logit[r] = (float)acc;
    }
    __syncthreads();
    if (wave == 0) {
        const float l = s_logit[lane];
        if (P.logits) P.logits[(int64_t)t * kRouted + lane] = l;
        wave_softmax_topk(l, kRouted, kTopK, P.scaling, s_ids, s_w, P.bias);
        // lanes < k read slots written by other lanes of this same wave
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
        if (lane < kTopK) {
            P.ids[(int64_t)t * kTopK + lane] = s_ids[lane];
            P.weights[(int64_t)t * kTopK + lane] = s_w[lane];
        }
    }
}

}  // namespace router

namespace fold {

// x_out = bf16(x + bf16(p_0 + p_1 + ... + p_{n-1})), the partials added in
// fp32 in index order (one thread per hidden element; x may equal x_out).
constexpr int kThreads = 256;
__global__ __launch_bounds__(kThreads) void residual_fold_kernel(const float* x,
                                                                 const float* partials,
                                                                 int n_partials, float* x_out) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    float acc = partials[i];
    for (int p = 1; p < n_partials; ++p) acc += partials[(int64_t)p * kHidden + i];
    x_out[i] = bf16r(x[i] + bf16r(acc));
}

}  // namespace fold

namespace probe {

// Streaming read with the weight-load pattern of the MoE kernels: each wave
// reads 4 contiguous 1 KB wave-loads (16-byte non-temporal loads per lane)
// per step, grid-stride. The XOR of everything read is written only if it
// equals an improbable constant, so the loads cannot be dropped.
constexpr int kThreads = 256;
constexpr int kDepth = 4;
__global__ __launch_bounds__(kThreads) void stream_read_kernel(const u32x4* __restrict__ p,
                                                               size_t n16, uint32_t* sink) {
    const int lane = threadIdx.x & (kLanes - 1);
    const size_t wave = (blockIdx.x * (size_t)kThreads + threadIdx.x) / kLanes;
    const size_t nwaves = (gridDim.x * (size_t)kThreads) / kLanes;
    const size_t tile = (size_t)kDepth * kLanes;
    uint32_t acc = 0;
    for (size_t t = wave * tile; t < n16; t += nwaves * tile) {
        u32x4 v[kDepth];
#pragma unroll
        for (int d = 0; d < kDepth; ++d) v[d] = ld_stream(p + t + d * kLanes + lane);
#pragma unroll
        for (int d = 0; d < kDepth; ++d) acc ^= v[d].x ^ v[d].y ^ v[d].z ^ v[d].w;
    }
    if (acc == 0x9e3779b9u) sink[0] = acc;
}

}  // namespace probe
}  // namespace fleet_moe

using namespace fleet_moe;

int fleet_moe_check_dims(const fleet_moe_dims* d) { return check_dims_impl(d); }
int fleet_moe_check_device(int min_cus) { return check_device_impl(min_cus); }
int fleet_moe_check_resident(const void* fn, int threads, int grid) {
    return check_resident_impl(fn, threads, grid);
}

static bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

extern "C" int fleet_moe_router_topk(const uint16_t* w_router, const float* x_norm,
                                     int32_t n_tokens, const float* logit_bias, float* logits,
                                     int32_t* ids, float* weights, const fleet_moe_dims* dims,
                                     hipStream_t stream) {
    if (int e = check_dims_impl(dims)) return e;
    if (!w_router || !x_norm || !ids || !weights || n_tokens < 1 || n_tokens > 65535)
        return FLEET_MOE_ERR_ARG;
    if (!aligned(w_router, 16) || !aligned(x_norm, 16) || !aligned(ids, 4) ||
        !aligned(weights, 4) || (logits && !aligned(logits, 4)) ||
        (logit_bias && !aligned(logit_bias, 4)))
        return FLEET_MOE_ERR_ARG;
    if (int e = check_device_impl(1)) return e;
    router::Params P;
    P.router = reinterpret_cast<const u32x4*>(w_router);
    P.x = x_norm;
    P.bias = logit_bias;
    P.logits = logits;
    P.ids = ids;
    P.weights = weights;
    P.scaling = dims->routed_scaling;
    hipLaunchKernelGGL(router::router_topk_kernel, dim3(n_tokens), dim3(router::kThreads), 0,
                       stream, P);
    return (int)hipGetLastError();
}

extern "C" int fleet_moe_residual_fold(const float* x, const float* partials, int32_t n_partials,
                                       float* x_out, const fleet_moe_dims* dims,
                                       hipStream_t stream) {
    if (int e = check_dims_impl(dims)) return e;
    if (!x || !partials || !x_out || n_partials < 1 || n_partials > 64 || !aligned(x, 4) ||
        !aligned(partials, 4) || !aligned(x_out, 4))
        return FLEET_MOE_ERR_ARG;
    if (int e = check_device_impl(1)) return e;
    hipLaunchKernelGGL(fold::residual_fold_kernel, dim3(kHidden / fold::kThreads),
                       dim3(fold::kThreads), 0, stream, x, partials, n_partials, x_out);
    return (int)hipGetLastError();
}

extern "C" int fleet_moe_stream_read(const void* buf, size_t bytes, uint32_t* sink,
                                     hipStream_t stream) {
    if (!buf || !sink || !aligned(buf, 16) || !aligned(sink, 4) || bytes == 0 ||
        bytes % (16 * kLanes * probe::kDepth) != 0)
        return FLEET_MOE_ERR_ARG;
    if (int e = check_device_impl(1)) return e;
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return (int)e;
    hipLaunchKernelGGL(probe::stream_read_kernel, dim3(2 * cus), dim3(probe::kThreads), 0, stream,
                       static_cast<const u32x4*>(buf), bytes / 16, sink);
    return (int)hipGetLastError();
}

extern "C" int fleet_moe_workspace_status(const void* workspace, uint32_t* status,
                                          hipStream_t stream) {
    if (!workspace || !status || !aligned(workspace, 256)) return FLEET_MOE_ERR_ARG;
    hipError_t e = hipMemcpyAsync(status, static_cast<const char*>(workspace) + 8,
                                  sizeof(uint32_t), hipMemcpyDeviceToHost, stream);
    if (e != hipSuccess) return (int)e;
    return (int)hipStreamSynchronize(stream);
}

extern "C" const char* fleet_moe_error_string(int code) {
    switch (code) {
        case 0: return "success";
        case FLEET_MOE_ERR_DIMS: return "fleet_moe: unsupported model shape";
        case FLEET_MOE_ERR_ARG: return "fleet_moe: null, misaligned or out-of-range argument";
        case FLEET_MOE_ERR_WORKSPACE: return "fleet_moe: workspace too small";
        case FLEET_MOE_ERR_DEVICE:
            return "fleet_moe: device is not a gfx950 with enough CUs to hold one workgroup of "
                   "the kernel on each";
        case FLEET_MOE_ERR_CAPACITY:
            return "fleet_moe: more tokens than the static scratch of the no-allocation entry "
                   "point holds";
        case FLEET_MOE_ERR_CAPTURE:
            return "fleet_moe: the first no-allocation call on a device sets up its scratch and "
                   "must not be made under graph capture";
        default: return hipGetErrorString((hipError_t)code);
    }
}

extern "C" int fleet_moe_abi_version(void) { return 101; }
