// Activation quantizer kernel and its C-ABI entry (the per-thread body and
// its reference semantics are in miq_xq.h).
#include "miq_xq.h"

namespace miq {

template <int LAYOUT>
__global__ __launch_bounds__(256) void xq_kernel(const float *__restrict__ x, const float *__restrict__ up,
                                                 int x_stride, int up_stride, int8_t *__restrict__ x8,
                                                 float *__restrict__ xmeta, int32_t *__restrict__ xsumq, int TB,
                                                 int G) {
    const int gid8 = blockIdx.x * blockDim.x + threadIdx.x;
    xq_lanes<LAYOUT>(x, up, x_stride, up_stride, x8, xmeta, xsumq, TB, G, gid8, (gid8 >> 3) < TB * G);
}

__global__ __launch_bounds__(256) void expf_range_kernel(uint32_t first, uint32_t count, float *__restrict__ y) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i < count) y[i] = expf_libm(__builtin_bit_cast(float, first + i));
}

int launch_xq(hipStream_t stream, const float *x, const float *up, int x_stride, int up_stride, int8_t *x8,
              float *xmeta, int32_t *xsumq, int TB, int K, int layout) {
    if (!x || !x8 || !xmeta || (!xsumq && layout == 0) || TB <= 0 || K <= 0 || K % (layout ? 64 : 32) ||
        x_stride < K || (up && up_stride < K) || layout < 0 || layout > 2 || (layout == 2 && K % 256)) {
        set_error("miq_xq: bad arguments (TB=%d K=%d x_stride=%d)", TB, K, x_stride);
        return MIQ_EINVAL;
    }
    if (((uintptr_t)x | (uintptr_t)(up ? up : x)) & 15 || (x_stride | (up ? up_stride : 0)) & 3 ||
        ((uintptr_t)x8 & 15) || ((uintptr_t)xmeta & (layout ? 15 : 7)) || ((uintptr_t)xsumq & 7)) {
        set_error("miq_xq: misaligned buffers (x/up 16 B with strides %% 4, x8 16 B, xmeta/xsumq 8 B)");
        return MIQ_UNSUPPORTED;
    }
    const int G = K / 32;
    const long n8 = (long)TB * G * 8;  // eight lanes per (token, group)
    if (n8 >= (1L << 31)) {
        set_error("miq_xq: %d tokens x %d groups is too large", TB, G);
        return MIQ_UNSUPPORTED;
    }
    const dim3 grid((unsigned)((n8 + 255) / 256)), block(256);
    if (layout == 0)
        hipLaunchKernelGGL(xq_kernel<0>, grid, block, 0, stream, x, up, x_stride, up_stride, x8, xmeta, xsumq, TB, G);
    else if (layout == 1)
        hipLaunchKernelGGL(xq_kernel<1>, grid, block, 0, stream, x, up, x_stride, up_stride, x8, xmeta, xsumq, TB, G);
    else
        hipLaunchKernelGGL(xq_kernel<2>, grid, block, 0, stream, x, up, x_stride, up_stride, x8, xmeta, xsumq, TB, G);
    return check_launch("miq_xq");
}

}  // namespace miq

extern "C" int miq_xq(hipStream_t stream, const float *x, const float *up, int x_stride, int up_stride, int8_t *x8,
                      float *xmeta, int32_t *xsumq, int TB, int K) {
    return miq::launch_xq(stream, x, up, x_stride, up_stride, x8, xmeta, xsumq, TB, K, 0);
}

extern "C" int miq_expf_range(hipStream_t stream, uint32_t first, uint32_t count, float *y) {
    if (!y || (uint64_t)first + count > 0x100000000ull) {
        miq::set_error("miq_expf_range: null output or range past 2^32");
        return MIQ_EINVAL;
    }
    if (!count) return MIQ_OK;
    hipLaunchKernelGGL(miq::expf_range_kernel, dim3((count + 255) / 256), dim3(256), 0, stream, first, count, y);
    return miq::check_launch("miq_expf_range");
}
