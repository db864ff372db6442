// Synthetic data on the device: N(0,1) samples from a counter-based SplitMix64 stream and
// Box-Muller, so any element of any tensor can be produced without generating the ones before it.
// Sample definition (shared with the CPU twin used by the tests):
//   key   = SplitMix64 output of state (seed ^ stream * golden)
//   pair p: o1 = mix(key + (2p+1)*golden), o2 = mix(key + (2p+2)*golden)
//           u1 = ((o1 >> 11) + 0.5) * 2^-53, u2 = (o2 >> 11) * 2^-53
//           element 2p = r cos(2 pi u2), element 2p+1 = r sin(2 pi u2), r = sqrt(-2 ln u1)
//   value = (float)(offset + scale * z), then round-to-nearest-even to bf16 when asked.
// The double-precision log/sin/cos here and in the host libm may differ in their last bit, which
// reaches the stored f32/bf16 value only in rare rounding-boundary cases; tests that compare the
// two paths read the device data back instead of regenerating it.
#include <math.h>

#include "rbt2_internal.h"

namespace rbt {
namespace {

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;

__host__ __device__ inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ inline void store(void *dst, int dtype, uint64_t i, double z, float scale, float offset) {
    const float v = (float)((double)offset + (double)scale * z);
    if (dtype == RBT_DT_F32) {
        static_cast<float *>(dst)[i] = v;
    } else {
        uint32_t u = __float_as_uint(v);
        uint16_t h;
        if (v != v) {
            h = 0x7FC0;
        } else {
            u += 0x7FFFu + ((u >> 16) & 1u);
            h = (uint16_t)(u >> 16);
        }
        static_cast<uint16_t *>(dst)[i] = h;
    }
}

__global__ void fill_normal_kernel(void *dst, int dtype, uint64_t n, uint64_t key, uint64_t first, float scale,
                                   float offset) {
    const uint64_t g0 = first, g1 = first + n;
    const uint64_t p0 = g0 >> 1, p1 = (g1 + 1) >> 1;
    const uint64_t step = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t p = p0 + (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; p < p1; p += step) {
        const uint64_t o1 = mix64(key + (2 * p + 1) * kGolden);
        const uint64_t o2 = mix64(key + (2 * p + 2) * kGolden);
        const double u1 = ((double)(o1 >> 11) + 0.5) * (1.0 / 9007199254740992.0);
        const double u2 = (double)(o2 >> 11) * (1.0 / 9007199254740992.0);
        const double r = sqrt(-2.0 * log(u1));
        const double th = 6.283185307179586 * u2;
        const uint64_t ga = 2 * p, gb = 2 * p + 1;
        if (ga >= g0 && ga < g1) store(dst, dtype, ga - g0, r * cos(th), scale, offset);
        if (gb >= g0 && gb < g1) store(dst, dtype, gb - g0, r * sin(th), scale, offset);
    }
}

}  // namespace

hipError_t launch_fill_normal(const Launch &L, void *dst, int dtype, uint64_t n, uint64_t seed, uint64_t stream,
                              uint64_t first, float scale, float offset) {
    if (n == 0) return hipSuccess;
    const uint64_t key = mix64((seed ^ (stream * kGolden)) + kGolden);
    const uint64_t pairs = (n + 2) / 2;
    uint64_t blocks = (pairs + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    return launch(L, fill_normal_kernel, dim3((unsigned)blocks), dim3(256), 0, dst, dtype, n, key, first, scale,
                  offset);
}

}  // namespace rbt
