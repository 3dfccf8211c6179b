// C++ host layer over libmiq's C ABI, shaped like the reference's backend
// interface for the quantized-matmul path so C++ callers keep their call
// sites: the segment descriptor `gemv_seg` (src/backend/gpu/kernels/kernels.h:44-81),
// the `compute_backend` methods xq / i8_gemv / i8_gemm and the multi-segment
// decode call (src/backend/backend.h:104-121), the bool launchers of the GPU
// kernel library (kernels.h: false = shape not served, the caller falls back)
// and the MoE host entry points' argument order (cpu_moe_route / cpu_moe_reduce,
// src/backend/cpu/cpu_types.h:195-209).
//
// Differences a caller sees: a hipStream_t takes the place of the sycl::queue;
// `float2` is a plain {x, y} pair with sycl::float2's layout; an unsupported
// shape makes the methods throw miq::unsupported (a std::runtime_error), other
// failures std::runtime_error with the library's message.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <memory>
#include <stdexcept>
#include <string>

#include "miq.h"

namespace miq {

struct float2 {
    float x, y;
};
static_assert(sizeof(float2) == 8, "float2 must match sycl::float2 / xmeta pairs");

// Per-step device scalars of the reference (unused on this path: the integer
// kernels take their sizes from the arguments).
struct step_info;

// One GEMV output segment; the integer-path fields of the reference's gemv_seg.
struct gemv_seg {
    const void *w = nullptr;       // GGUF blocks [n_rows][K/QK] on the device
    uint32_t type = 0;             // ggml type of w (Q4_K 12, Q5_K 13, Q6_K 14, Q8_0 8)
    int32_t K = 0;                 // input length
    int32_t n_rows = 0;            // output rows
    int32_t dev = 0;               // backend device index (kept for layout parity)
    const float *x = nullptr;      // fp32 activations, row stride x_stride
    int32_t x_stride = 0;
    const float *act_up = nullptr; // non-null: x is activated as silu(x)*act_up
    float *out = nullptr;          // out[t*out_stride + row]
    int32_t out_stride = 0;
    const float *residual = nullptr;
    float alpha = 1.0f;
    const int8_t *x8 = nullptr;    // quantized activation (xq's output)
    const float2 *xmeta = nullptr; // {scale, 0} per (group, token)
    const int32_t *xsumq = nullptr;
    bool i8 = true;                // the integer path (always, here)
};

class unsupported : public std::runtime_error {
  public:
    explicit unsupported(const std::string &what) : std::runtime_error(what) {}
};

// The routed-expert banks (the integer fields of cpu_moe / the GPU moe_banks).
struct moe_banks {
    const void *gate = nullptr, *up = nullptr, *down = nullptr;
    uint32_t gate_type = 12, up_type = 12, down_type = 12;
    size_t gate_plane = 0, up_plane = 0, down_plane = 0;  // bytes of one expert in each bank
    int n_embd = 0, n_ff_exp = 0, n_expert = 0;
};

// The quantized-matmul slice of compute_backend, on one device and stream.
struct compute_backend {
    virtual ~compute_backend() = default;
    virtual const char *name() const = 0;

    // backend.h:104-105: quantize TB rows of K values (silu(x)*up with up)
    virtual void xq(const float *x, const float *up, int x_stride, int up_stride, int8_t *x8, float2 *xmeta,
                    int32_t *xsumq, const step_info *info, int TB, int K) = 0;
    // backend.h:113-114: integer GEMV (one token) / GEMM (TB tokens) on the
    // activation the segment's x8/xmeta/xsumq hold
    virtual void i8_gemv(const gemv_seg &s) = 0;
    virtual void i8_gemm(const gemv_seg &s, int TB) = 0;
    // backend.h:120-121 / kernels.h:216-219: every segment of a call (one K,
    // segs[0]'s activation) in one launch at decode sizes
    virtual void i8_gemv_multi(const gemv_seg *segs, int n_segs, int TB) = 0;
    // kernels.h:216-236: the activation quantizer fused with the GEMV (x / act_up of the segment)
    virtual void quant_gemm(const gemv_seg &s, int TB) = 0;

    // MoE (cpu_types.h:195-209 argument order; device pointers): route over
    // given logits (gate_inp == nullptr) or an fp32 router matrix, the routed
    // experts (unweighted acc rows), the weighted reduce
    virtual void moe_route(const float *x, int x_stride, const float *gate_inp, int n_tok, int n_embd, int n_expert,
                           int top_k, float *logits, int32_t *ids, float *wts) = 0;
    virtual void moe_experts(const moe_banks &M, const float *x, int x_stride, int n_tok, int top_k,
                             const int32_t *ids, float *acc, int acc_stride) = 0;
    virtual void moe_reduce(const float *acc, const float *wts, int top_k, int n_tok, int n_embd, int acc_stride,
                            float *out, int out_stride) = 0;

    virtual void synchronize() = 0;
};

// The GPU backend over libmiq on `stream` (the reference: make_gpu_backend(sycl::queue &)).
std::unique_ptr<compute_backend> make_gpu_backend(hipStream_t stream);

// Launcher forms (kernels.h): false when the shape is not served (nothing is
// launched; miq_last_error() says why), throw on any other failure.
bool i8_gemv_launch(hipStream_t stream, const gemv_seg &s);
bool i8_gemm_launch(hipStream_t stream, const gemv_seg &s, int TB);

// The C ABI's segment for a gemv_seg (field for field).
miq_seg to_miq(const gemv_seg &s);

}  // namespace miq
