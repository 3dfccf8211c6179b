// The C++ host layer over libmiq (see miq_backend.hpp).
#include "miq_backend.hpp"

#include <vector>

namespace miq {

miq_seg to_miq(const gemv_seg &s) {
    miq_seg m{};
    m.w = s.w;
    m.type = s.type;
    m.K = s.K;
    m.n_rows = s.n_rows;
    m.x = s.x;
    m.x_stride = s.x_stride;
    m.act_up = s.act_up;
    m.out = s.out;
    m.out_stride = s.out_stride;
    m.residual = s.residual;
    m.alpha = s.alpha;
    m.x8 = s.x8;
    m.xmeta = reinterpret_cast<const float *>(s.xmeta);
    m.xsumq = s.xsumq;
    return m;
}

namespace {

// MIQ_OK -> return; MIQ_UNSUPPORTED -> unsupported; anything else -> runtime_error
void check(int rc, const char *what) {
    if (rc == MIQ_OK) return;
    const std::string msg = std::string(what) + ": " + miq_last_error();
    if (rc == MIQ_UNSUPPORTED) throw unsupported(msg);
    throw std::runtime_error(msg);
}

class gpu_backend final : public compute_backend {
  public:
    explicit gpu_backend(hipStream_t stream) : stream_(stream) {}
    ~gpu_backend() override {
        // the caller's work on stream_ has finished by the time it destroys the backend
        if (ws_) (void)hipFree(ws_);
        for (void *p : retired_) (void)hipFree(p);
    }
    const char *name() const override { return "miq (gfx950)"; }

    void xq(const float *x, const float *up, int x_stride, int up_stride, int8_t *x8, float2 *xmeta, int32_t *xsumq,
            const step_info *, int TB, int K) override {
        check(miq_xq(stream_, x, up, x_stride, up_stride, x8, reinterpret_cast<float *>(xmeta), xsumq, TB, K),
              "xq");
    }
    void i8_gemv(const gemv_seg &s) override {
        const miq_seg m = to_miq(s);
        check(miq_i8_gemv(stream_, &m), "i8_gemv");
    }
    void i8_gemm(const gemv_seg &s, int TB) override {
        const miq_seg m = to_miq(s);
        check(miq_i8_gemm(stream_, &m, TB), "i8_gemm");
    }
    void i8_gemv_multi(const gemv_seg *segs, int n_segs, int TB) override {
        if (n_segs < 1 || n_segs > 8) throw std::invalid_argument("i8_gemv_multi: 1..8 segments");
        miq_seg m[8];
        for (int i = 0; i < n_segs; i++) m[i] = to_miq(segs[i]);
        check(miq_i8_gemv_multi(stream_, m, n_segs, TB), "i8_gemv_multi");
    }
    void quant_gemm(const gemv_seg &s, int TB) override {
        const miq_seg m = to_miq(s);
        check(miq_quant_gemm(stream_, &m, TB), "quant_gemm");
    }
    void moe_route(const float *x, int x_stride, const float *gate_inp, int n_tok, int n_embd, int n_expert,
                   int top_k, float *logits, int32_t *ids, float *wts) override {
        check(miq_moe_route(stream_, x, x_stride, gate_inp, n_tok, n_embd, n_expert, top_k, logits, ids, wts),
              "moe_route");
    }
    void moe_experts(const moe_banks &B, const float *x, int x_stride, int n_tok, int top_k, const int32_t *ids,
                     float *acc, int acc_stride) override {
        miq_moe M{};
        M.gate = B.gate;
        M.up = B.up;
        M.down = B.down;
        M.gate_type = B.gate_type;
        M.up_type = B.up_type;
        M.down_type = B.down_type;
        M.gate_plane = B.gate_plane;
        M.up_plane = B.up_plane;
        M.down_plane = B.down_plane;
        M.n_embd = B.n_embd;
        M.n_ff = B.n_ff_exp;
        M.n_expert = B.n_expert;
        const size_t need = miq_moe_workspace_bytes(&M, n_tok, top_k);
        if (!need) throw std::invalid_argument("moe_experts: bad shape");
        if (need > ws_bytes_) {
            // The backend owns its workspace and grows it between calls.  Allocation
            // inside a recorded graph is illegal (kernels.h:585-594), so a capturing
            // stream gets `unsupported` and the caller warms the shape up first.  A
            // grown-out buffer is kept until the backend is destroyed: queued work and
            // graphs captured earlier still point at it, so nothing waits and nothing
            // they read is freed.
            hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
            if (hipStreamIsCapturing(stream_, &cs) != hipSuccess)
                throw std::runtime_error("moe_experts: hipStreamIsCapturing");
            if (cs != hipStreamCaptureStatusNone)
                throw unsupported("moe_experts: the workspace must grow while the stream captures a graph");
            void *p = nullptr;
            if (hipMalloc(&p, need) != hipSuccess) throw std::runtime_error("moe_experts: workspace allocation");
            if (ws_) retired_.push_back(ws_);
            ws_ = p;
            ws_bytes_ = need;
        }
        check(miq_moe_experts(stream_, &M, x, x_stride, n_tok, top_k, ids, acc, acc_stride, ws_, ws_bytes_),
              "moe_experts");
    }
    void moe_reduce(const float *acc, const float *wts, int top_k, int n_tok, int n_embd, int acc_stride, float *out,
                    int out_stride) override {
        check(miq_moe_reduce(stream_, acc, wts, top_k, n_tok, n_embd, acc_stride, out, out_stride), "moe_reduce");
    }
    void synchronize() override {
        if (hipStreamSynchronize(stream_) != hipSuccess) throw std::runtime_error("synchronize: hipStreamSynchronize");
    }

  private:
    hipStream_t stream_;
    void *ws_ = nullptr;
    size_t ws_bytes_ = 0;
    std::vector<void *> retired_;
};

}  // namespace

std::unique_ptr<compute_backend> make_gpu_backend(hipStream_t stream) { return std::make_unique<gpu_backend>(stream); }

bool i8_gemv_launch(hipStream_t stream, const gemv_seg &s) {
    const miq_seg m = to_miq(s);
    const int rc = miq_i8_gemv(stream, &m);
    if (rc == MIQ_UNSUPPORTED) return false;
    check(rc, "i8_gemv_launch");
    return true;
}

bool i8_gemm_launch(hipStream_t stream, const gemv_seg &s, int TB) {
    const miq_seg m = to_miq(s);
    const int rc = miq_i8_gemm(stream, &m, TB);
    if (rc == MIQ_UNSUPPORTED) return false;
    check(rc, "i8_gemm_launch");
    return true;
}

}  // namespace miq
