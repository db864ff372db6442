// Internal declarations shared by the gfx950 kernels and the C-ABI layer (not installed).
#pragma once

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

// ---- launchers (each returns hipSuccess or the launch error) ----

// Router logits in the engine's exact order + softmax + top-k + combine weights, one token per
// grid row; the last block of each token finishes the softmax/top-k (counters[t] must be 0 on
// entry and are left 0). probs: [T][E] workspace.
hipError_t launch_router(hipStream_t s, int order, int dtype, const float *xb, const void *W, const float *bias, int T,
                         int E, int D, int K, int norm_topk, float *probs, unsigned *counters, int32_t *routing,
                         float *weights);

// Per-(token, slot) GEMV form of the expert FFN (decode and small batches).
hipError_t launch_gateup_gemv(hipStream_t s, int dtype, const void *experts, uint64_t stride, const int32_t *routing,
                              const float *xb, int T, int K, int D, int H, float *hbuf);
hipError_t launch_down_combine(hipStream_t s, int dtype, const void *experts, uint64_t stride, const int32_t *routing,
                               const float *weights, const float *hbuf, int T, int K, int D, int H, float *x_inout,
                               float *moe_out);

// Dense matvec (one row per wave).
hipError_t launch_matvec(hipStream_t s, int dtype, const void *W, const float *x, float *out, int rows, int cols);

// Synthetic normal fill (SplitMix64 + Box-Muller), see rbt_hip_fill_normal.
hipError_t launch_fill_normal(hipStream_t s, void *dst, int dtype, uint64_t n, uint64_t seed, uint64_t stream,
                              uint64_t first, float scale, float offset);

}  // namespace rbt
