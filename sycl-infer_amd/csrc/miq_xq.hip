// Activation quantizer: fp32 rows -> per-32-group int8 codes, f16-truncated
// scale and the two per-16 code sums.
//
// Semantics of cpu_xq (src/backend/cpu/kernels/xq.cpp:10-50), bit for bit:
//   mx = max|v|; inv = 127/mx (IEEE division); q = clamp(roundf(v*inv), +-127)
//   (round half away from zero); scale = f16trunc(mx/127) as fp32, 0 for an
//   all-zero group; s0 = sum q[0..15], s1 = sum q[16..31].
// With `up` the value is silu(x)*up; silu uses the device expf, so that form
// can differ from the host's libm in the last ulp (and then by one code).
#include "miq_common.h"

namespace miq {

__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

// One thread per (token, group): 128 contiguous input bytes, 32 output bytes.
__global__ __launch_bounds__(256) void xq_kernel(const float *__restrict__ x, const float *__restrict__ up,
                                                 int x_stride, int up_stride, int8_t *__restrict__ x8,
                                                 float *__restrict__ xmeta, int32_t *__restrict__ xsumq, int TB,
                                                 int G) {
    const int gid = blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= TB * G) return;
    const int t = gid / G;
    const int g = gid - t * G;
    const float4 *src = reinterpret_cast<const float4 *>(x + (size_t)t * x_stride + g * 32);
    float v[32];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 a = src[i];
        v[4 * i + 0] = a.x;
        v[4 * i + 1] = a.y;
        v[4 * i + 2] = a.z;
        v[4 * i + 3] = a.w;
    }
    if (up) {
        const float4 *u = reinterpret_cast<const float4 *>(up + (size_t)t * up_stride + g * 32);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 b = u[i];
            v[4 * i + 0] = silu(v[4 * i + 0]) * b.x;
            v[4 * i + 1] = silu(v[4 * i + 1]) * b.y;
            v[4 * i + 2] = silu(v[4 * i + 2]) * b.z;
            v[4 * i + 3] = silu(v[4 * i + 3]) * b.w;
        }
    }
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        const float a = fabsf(v[i]);
        mx = mx < a ? a : mx;
    }
    const float inv = mx > 0.0f ? 127.0f / mx : 0.0f;
    int s0 = 0, s1 = 0;
    uint32_t packed[8];
#pragma unroll
    for (int w = 0; w < 8; w++) {
        uint32_t word = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            float r = roundf(v[4 * w + b] * inv);
            r = r < 127.0f ? r : 127.0f;
            r = -127.0f > r ? -127.0f : r;
            const int q = (int)r;
            if (4 * w + b < 16) s0 += q; else s1 += q;
            word |= ((uint32_t)q & 0xFFu) << (8 * b);
        }
        packed[w] = word;
    }
    const size_t gi = (size_t)g * TB + t;
    uint4 *dst = reinterpret_cast<uint4 *>(x8 + gi * 32);
    dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    dst[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
    const float scale = mx > 0.0f ? mx / 127.0f : 0.0f;
    reinterpret_cast<float2 *>(xmeta)[gi] = make_float2(h2f(f2h_trunc(scale)), 0.0f);
    reinterpret_cast<int2 *>(xsumq)[gi] = make_int2(s0, s1);
}

int launch_xq(hipStream_t stream, const float *x, const float *up, int x_stride, int up_stride, int8_t *x8,
              float *xmeta, int32_t *xsumq, int TB, int K) {
    if (!x || !x8 || !xmeta || !xsumq || TB <= 0 || K <= 0 || K % 32 || x_stride < K || (up && up_stride < K)) {
        set_error("miq_xq: bad arguments (TB=%d K=%d x_stride=%d)", TB, K, x_stride);
        return MIQ_EINVAL;
    }
    if (((uintptr_t)x | (uintptr_t)(up ? up : x)) & 15 || (x_stride | (up ? up_stride : 0)) & 3 ||
        ((uintptr_t)x8 & 15) || ((uintptr_t)xmeta & 7) || ((uintptr_t)xsumq & 7)) {
        set_error("miq_xq: misaligned buffers (x/up 16 B with strides %% 4, x8 16 B, xmeta/xsumq 8 B)");
        return MIQ_UNSUPPORTED;
    }
    const int G = K / 32;
    const int n = TB * G;
    hipLaunchKernelGGL(xq_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, x, up, x_stride, up_stride, x8,
                       xmeta, xsumq, TB, G);
    return check_launch("miq_xq");
}

}  // namespace miq

extern "C" int miq_xq(hipStream_t stream, const float *x, const float *up, int x_stride, int up_stride, int8_t *x8,
                      float *xmeta, int32_t *xsumq, int TB, int K) {
    return miq::launch_xq(stream, x, up, x_stride, up_stride, x8, xmeta, xsumq, TB, K);
}
