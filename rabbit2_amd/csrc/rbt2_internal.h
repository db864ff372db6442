// Internal declarations shared by the gfx950 kernels and the C-ABI layer (not installed).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/rbt2_hip.h"

namespace rbt {

constexpr int kWave = 64;  // CDNA wavefront width

// bf16 storage -> f32 is exact: the 16 stored bits are the high half of the f32 (rabbit2.c:304-309).
__device__ __forceinline__ float bf16_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t pair) { return __uint_as_float(pair & 0xFFFF0000u); }

template <int DT>
__device__ __forceinline__ float load_w(const void *W, size_t i) {
    if constexpr (DT == RBT_DT_F32) {
        return static_cast<const float *>(W)[i];
    } else {
        return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t *>(W)[i]) << 16);
    }
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// 16-byte streaming load (weights are read once per layer; the non-temporal hint keeps them from
// displacing reused data in the caches).
__device__ __forceinline__ u32x4 ld_stream_u4(const void *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
}
__device__ __forceinline__ f32x4 ld_stream_f4(const void *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
}
__device__ __forceinline__ f32x4 ld_f4(const float *p) { return *reinterpret_cast<const f32x4 *>(p); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// Where and how a kernel is launched: the stream, and optionally a pair of events that the runtime
// stamps with the kernel's own start and end (hipExtLaunchKernel), used by the profiling mode.
struct Launch {
    hipStream_t s = nullptr;
    hipEvent_t start = nullptr, stop = nullptr;
};

template <typename F, typename... Args>
inline hipError_t launch(const Launch &L, F kernel, dim3 grid, dim3 block, uint32_t shmem, Args... args) {
    hipExtLaunchKernelGGL(kernel, grid, block, shmem, L.s, L.start, L.stop, 0, args...);
    return hipGetLastError();
}

// ---- launchers (each returns hipSuccess or the launch error) ----

// Router logits in the engine's exact order (logits kernel, launch context L), then softmax + top-k +
// combine weights (one block per token, context Lk). probs: [T][E] workspace (logits, then
// probabilities).
hipError_t launch_router(const Launch &L, const Launch &Lk, int order, int dtype, const float *xb, const void *W,
                         const float *bias, int T, int E, int D, int K, int norm_topk, float *probs,
                         int32_t *routing, float *weights);

// Per-(token, slot) GEMV form of the expert FFN (decode and small batches).
hipError_t launch_gateup_gemv(const Launch &L, int dtype, const void *experts, uint64_t stride, const int32_t *routing,
                              const float *xb, int T, int K, int D, int H, float *hbuf);
hipError_t launch_down_combine(const Launch &L, int dtype, const void *experts, uint64_t stride, const int32_t *routing,
                               const float *weights, const float *hbuf, int T, int K, int D, int H, float *x_inout,
                               float *moe_out);

// The same expert FFN specialised for whole-wave-step row lengths (the OLMoE shape among them):
// every load of a wave is issued before the first wait. Lg/Ld: launch contexts of the gate/up and
// down kernels.
bool experts_decode_supported(int dtype, int T, int K, int D, int H, const void *experts, uint64_t stride,
                              const float *xb, const float *hbuf);
hipError_t launch_experts_decode(const Launch &Lg, const Launch &Ld, int dtype, const void *experts, uint64_t stride,
                                 const int32_t *routing, const float *weights, const float *xb, float *hbuf, int T,
                                 int K, int D, int H, float *x_inout, float *moe_out);

// Dense matvec (one row per wave).
hipError_t launch_matvec(const Launch &L, int dtype, const void *W, const float *x, float *out, int rows, int cols);

// Synthetic normal fill (SplitMix64 + Box-Muller), see rbt_hip_fill_normal.
hipError_t launch_fill_normal(const Launch &L, void *dst, int dtype, uint64_t n, uint64_t seed, uint64_t stream,
                              uint64_t first, float scale, float offset);

}  // namespace rbt
