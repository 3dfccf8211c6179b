// Compute-only ceilings of the prefill GEMM's inner step on gfx950: no
// memory traffic, operands held in registers (an empty asm keeps the compiler
// from hoisting them out of the loop).  Each wave owns a 64-row x 64-token
// output tile (4 x 4 tiles of 16 x 16) and runs `groups` 32-value K groups.
// Per group and tile the variants issue:
//   f16_epi   1 fp16 MFMA 16x16x32 (sum sc*I of the group, exact) + 4 fp32 fma  (ab += sx * C)
//   i8_epi    1 int8 MFMA 16x16x32 (the group's int32 dot)  + 4 x (cvt, mul, fma) (ab += sx*dsc * I)
//   f16_2mfma 2 fp16 MFMAs accumulating in place (activation pre-scaled by sx, split hi/lo), no VALU
//   f16_pure  1 fp16 MFMA accumulating in place (the fp16 rate, no epilogue)
//   i8_pure   1 int8 MFMA 16x16x64 per two groups, accumulating in place (the int8 rate)
//   f16_pipe  f16_epi with the epilogue one group behind the MFMAs (two sets of results)
//   f16_indep f16_pure plus 4 fp32 fma per tile that do not depend on the MFMAs (does
//             VALU work issue under the matrix core's?)
// Ops are counted as 2*M*N*K of the GEMM (int8-equivalent), so every variant
// is priced against the same work.  Usage: mfma_ceiling [groups] [wg_per_cu] [waves_per_wg]
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef int i4 __attribute__((ext_vector_type(4)));
typedef int i2 __attribute__((ext_vector_type(2)));
typedef long l2 __attribute__((ext_vector_type(2)));

#define KEEP(r_) asm volatile("" : "+v"((r_).x), "+v"((r_).y), "+v"((r_).z), "+v"((r_).w))

template <int V>
__global__ __launch_bounds__(512) void ceiling(const uint4 *src, float *dst, int groups) {
    const int lane = threadIdx.x & 63;
    uint4 ra[4], rb[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        ra[i] = src[(lane + 64 * i) & 255];
        rb[i] = src[(lane + 64 * i + 7) & 255];
    }
    float sxs[4], dsc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        sxs[i] = __builtin_bit_cast(float, (ra[i].x & 0x007FFFFFu) | 0x3F800000u);
#pragma unroll
        for (int v = 0; v < 4; v++) dsc[i][v] = __builtin_bit_cast(float, (rb[v].y & 0x007FFFFFu) | 0x3F000000u);
    }
    f4 ab[4][4];
    i4 ib[4][4];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++) {
            ab[a][b] = f4{0, 0, 0, 0};
            ib[a][b] = i4{0, 0, 0, 0};
        }
    f4 cq[2][16];
#pragma unroll
    for (int p = 0; p < 16; p++) cq[0][p] = cq[1][p] = f4{0, 0, 0, 0};
    for (int g = 0; g < groups; g++) {
        h8 av[4], bv[4], al[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            KEEP(ra[i]);
            KEEP(rb[i]);
            av[i] = __builtin_bit_cast(h8, ra[i]);
            bv[i] = __builtin_bit_cast(h8, rb[i]);
            al[i] = __builtin_bit_cast(h8, uint4{rb[i].y, rb[i].x, ra[i].w, ra[i].z});
        }
        if constexpr (V == 0) {
#pragma unroll
            for (int p = 0; p < 16; p++) {
                const f4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[p >> 2], bv[p & 3], f4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 4; v++) ab[p >> 2][p & 3][v] = __builtin_fmaf(sxs[p & 3], c[v], ab[p >> 2][p & 3][v]);
            }
        } else if constexpr (V == 1) {
#pragma unroll
            for (int p = 0; p < 16; p++) {
                const l2 x = __builtin_bit_cast(l2, ra[p >> 2]), y = __builtin_bit_cast(l2, rb[p & 3]);
                const i4 c = __builtin_amdgcn_mfma_i32_16x16x32_i8(x[0], y[0], i4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 4; v++)
                    ab[p >> 2][p & 3][v] = __builtin_fmaf(sxs[p & 3] * dsc[p >> 2][v], (float)c[v], ab[p >> 2][p & 3][v]);
            }
        } else if constexpr (V == 2) {
#pragma unroll
            for (int p = 0; p < 16; p++) {
                ab[p >> 2][p & 3] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[p >> 2], bv[p & 3], ab[p >> 2][p & 3], 0, 0, 0);
                ab[p >> 2][p & 3] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[p >> 2], bv[p & 3], ab[p >> 2][p & 3], 0, 0, 0);
            }
        } else if constexpr (V == 5) {
            // f16_pure plus the same 64 fmas per group on registers the MFMAs do not touch
#pragma unroll
            for (int p = 0; p < 16; p++) {
                ab[p >> 2][p & 3] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[p >> 2], bv[p & 3], ab[p >> 2][p & 3], 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 4; v++)
                    dsc[p >> 2][v] = __builtin_fmaf(sxs[p & 3], dsc[p >> 2][v], dsc[(p + 1) & 3][v]);
            }
        } else if constexpr (V == 6) {
            // f16_epi software-pipelined by one group: this group's 16 MFMAs are issued
            // first, then the previous group's epilogue reads results that have landed
            // (two groups per iteration so both result sets stay in fixed registers)
            if (g & 1) continue;
#pragma unroll
            for (int p = 0; p < 16; p++)
                cq[0][p] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[p >> 2], bv[p & 3], f4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int p = 0; p < 16; p++)
#pragma unroll
                for (int v = 0; v < 4; v++) ab[p >> 2][p & 3][v] = __builtin_fmaf(sxs[p & 3], cq[1][p][v], ab[p >> 2][p & 3][v]);
#pragma unroll
            for (int p = 0; p < 16; p++)
                cq[1][p] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[p >> 2], bv[p & 3], f4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int p = 0; p < 16; p++)
#pragma unroll
                for (int v = 0; v < 4; v++) ab[p >> 2][p & 3][v] = __builtin_fmaf(sxs[(p + 1) & 3], cq[0][p][v], ab[p >> 2][p & 3][v]);
        } else if constexpr (V == 3) {
#pragma unroll
            for (int p = 0; p < 16; p++)
                ab[p >> 2][p & 3] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av[p >> 2], bv[p & 3], ab[p >> 2][p & 3], 0, 0, 0);
        } else {
            if (g & 1) continue;  // one 64-deep MFMA per two groups
#pragma unroll
            for (int p = 0; p < 16; p++)
                ib[p >> 2][p & 3] = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(i4, ra[p >> 2]),
                                                                         __builtin_bit_cast(i4, rb[p & 3]),
                                                                         ib[p >> 2][p & 3], 0, 0, 0);
        }
    }
    float s = 0;
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 4; b++)
#pragma unroll
            for (int v = 0; v < 4; v++) s += ab[a][b][v] + (float)ib[a][b][v] + dsc[a][v];
    dst[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

int main(int argc, char **argv) {
    const int groups = argc > 1 ? atoi(argv[1]) : 4096;
    const int wg_cu = argc > 2 ? atoi(argv[2]) : 2;
    const int waves = argc > 3 ? atoi(argv[3]) : 4;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, 0) != hipSuccess) return 2;
    const int cus = prop.multiProcessorCount, grid = cus * wg_cu, block = 64 * waves;
    uint4 *src;
    float *dst;
    (void)hipMalloc(&src, 256 * sizeof(uint4));
    (void)hipMalloc(&dst, (size_t)grid * block * sizeof(float));
    unsigned h[1024];
    for (int i = 0; i < 1024; i++) h[i] = 0x3C003C00u ^ (i * 2654435761u & 0x03FF03FFu);
    (void)hipMemcpy(src, h, sizeof(h), hipMemcpyHostToDevice);
    const char *names[7] = {"f16_epi", "i8_epi", "f16_2mfma", "f16_pure", "i8_pure", "f16_indep", "f16_pipe"};
    void (*kern[7])(const uint4 *, float *, int) = {ceiling<0>, ceiling<1>, ceiling<2>, ceiling<3>, ceiling<4>, ceiling<5>, ceiling<6>};
    hipEvent_t e0, e1;
    (void)hipEventCreate(&e0);
    (void)hipEventCreate(&e1);
    printf("%d CUs, %d workgroups of %d waves, %d groups of 32 per wave tile 64x64\n", cus, grid, waves, groups);
    for (int v = 0; v < 7; v++) {
        hipLaunchKernelGGL(kern[v], dim3(grid), dim3(block), 0, 0, src, dst, 64);
        (void)hipDeviceSynchronize();
        (void)hipEventRecord(e0, 0);
        for (int r = 0; r < 5; r++) hipLaunchKernelGGL(kern[v], dim3(grid), dim3(block), 0, 0, src, dst, groups);
        (void)hipEventRecord(e1, 0);
        (void)hipEventSynchronize(e1);
        float ms = 0;
        (void)hipEventElapsedTime(&ms, e0, e1);
        const double ops = 5.0 * grid * waves * (double)groups * 2.0 * 64 * 64 * 32;
        printf("%-10s %8.3f ms  %7.1f TOPS (int8-equivalent)  %5.1f %% of 5000\n", names[v], ms / 5, ops / (ms * 1e-3) / 1e12,
               ops / (ms * 1e-3) / 1e12 / 50.0);
    }
    return 0;
}
