// Seeded synthetic inputs generated on the device (benchmark and test data, not part of the
// projection path): block scales log-uniform in [2^lo, 2^hi], weights N(0,1)/scale quantised to
// e4m3 with saturation at +-448, activations N(0, stddev^2) rounded to bf16.
// Counter-based: element i of a stream with seed s depends only on (s, i), so any slice can be
// regenerated or checked independently of launch shape.
#include "pw_device.h"
#include "pw_launch.h"

namespace pw {

__device__ __forceinline__ uint64_t splitmix64(uint64_t z)
{
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// Two N(0,1) samples from one 64-bit counter hash (Box-Muller, f32).
__device__ __forceinline__ float2 normal2(uint64_t seed, uint64_t counter)
{
    const uint64_t h = splitmix64(seed ^ splitmix64(counter));
    const float u1 = ((float)(uint32_t)(h >> 40) + 0.5f) * (1.0f / 16777216.0f);  // (0, 1)
    const float u2 = (float)(uint32_t)((h >> 8) & 0xffffffu) * (1.0f / 16777216.0f);
    const float r = sqrtf(-2.0f * logf(u1));
    float sn, cs;
    sincosf(6.28318530717958647692f * u2, &sn, &cs);
    return make_float2(r * cs, r * sn);
}

__global__ void synth_fp8_kernel(uint8_t *__restrict__ w, const float *__restrict__ scales,
                                 uint64_t rows, uint64_t cols, uint64_t seed)
{
    const uint64_t quads = rows * cols / 4;
    const uint64_t scale_cols = cols / 128;
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < quads;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t e0 = i * 4;
        const uint64_t r = e0 / cols, c = e0 % cols;  // 4 | cols, so the quad stays in one row
        const float s = scales[(r / 128) * scale_cols + c / 128];
        const float2 a = normal2(seed, i * 2), b = normal2(seed, i * 2 + 1);
        const float z[4] = {a.x, a.y, b.x, b.y};
        uint32_t packed = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float v = z[j] / s;
            v = v < -448.f ? -448.f : (v > 448.f ? 448.f : v);
            packed |= (uint32_t)encode_e4m3fn_rne(v) << (8 * j);
        }
        *(uint32_t *)(w + e0) = packed;
    }
}

__global__ void synth_scales_kernel(float *__restrict__ s, uint64_t count, uint64_t seed, float lo,
                                    float hi)
{
    const uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x;
    if (i >= count)
        return;
    const uint64_t h = splitmix64(seed ^ splitmix64(i));
    const float u = (float)(uint32_t)(h >> 40) * (1.0f / 16777216.0f);
    s[i] = exp2f(lo + (hi - lo) * u);
}

__global__ void synth_normal_bf16_kernel(uint16_t *__restrict__ x, uint64_t count, uint64_t seed,
                                         float stddev)
{
    const uint64_t pairs = count / 2;
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < pairs;
         i += (uint64_t)gridDim.x * blockDim.x) {
        const float2 z = normal2(seed, i);
        x[2 * i] = bf16_bits(z.x * stddev);
        x[2 * i + 1] = bf16_bits(z.y * stddev);
    }
}

static int synth_grid(uint64_t work)
{
    const uint64_t g = (work + 255) / 256;
    return (int)(g < 262144 ? (g ? g : 1) : 262144);
}

void launch_synth_fp8(uint8_t *w, const float *scales, uint64_t rows, uint64_t cols, uint64_t seed,
                      hipStream_t stream)
{
    hipLaunchKernelGGL(synth_fp8_kernel, dim3(synth_grid(rows * cols / 4)), dim3(256), 0, stream, w,
                       scales, rows, cols, seed);
}

void launch_synth_scales(float *s, uint64_t count, uint64_t seed, float log2_lo, float log2_hi,
                         hipStream_t stream)
{
    hipLaunchKernelGGL(synth_scales_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0,
                       stream, s, count, seed, log2_lo, log2_hi);
}

void launch_synth_normal_bf16(uint16_t *x, uint64_t count, uint64_t seed, float stddev,
                              hipStream_t stream)
{
    hipLaunchKernelGGL(synth_normal_bf16_kernel, dim3(synth_grid(count / 2)), dim3(256), 0, stream,
                       x, count, seed, stddev);
}

}  // namespace pw
