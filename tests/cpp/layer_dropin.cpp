// layer_dropin.cpp -- HipGPT's attention sub-layer replayed through the
// drop-in C++ symbols of libhipgpt_attn.so, checked against the CPU oracle.
//
// The forward is the call sequence of TransformerLayer::self_attention_forward
// (src/transformer_layer.cpp:214-222): QKV projection with launch_matmul_add_bias
// into the [T][3E] buffer, launch_multihead_attention reading that buffer as
// planar [Q|K|V], output projection.  The backward is the attention step of
// TransformerLayer::backward (:285-286): launch_multihead_attention_backward on
// the forward's probs.  Every launcher runs on the null stream and the host
// reads results back with blocking hipMemcpy, as HipGPT does.  The program links
// only libhipgpt_attn.so (the library under test) and liboracle_attn.so (the
// checker); it includes nothing of this library but include/hip_kernels.h.
//
// Usage: layer_dropin B S E H   -> prints the max errors, exits 0 when every
// stage is within 1e-4 * max(1, max|want|) of the oracle, 1 otherwise.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "hip_kernels.h"

extern "C" {
#include "attn_oracle.h"
}

namespace {

#define HIP_OK(x)                                                                       \
    do {                                                                                \
        hipError_t e_ = (x);                                                            \
        if (e_ != hipSuccess) {                                                         \
            std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x,              \
                         hipGetErrorString(e_));                                        \
            std::exit(2);                                                               \
        }                                                                               \
    } while (0)

struct Dev {
    float* p = nullptr;
    size_t n = 0;
    explicit Dev(size_t n_) : n(n_) { HIP_OK(hipMalloc(&p, n * sizeof(float) + 4)); }
    ~Dev() { (void)hipFree(p); }
    void put(const std::vector<float>& h) { HIP_OK(hipMemcpy(p, h.data(), n * sizeof(float), hipMemcpyHostToDevice)); }
    std::vector<float> get() const {
        std::vector<float> h(n);
        HIP_OK(hipMemcpy(h.data(), p, n * sizeof(float), hipMemcpyDeviceToHost));
        return h;
    }
    // NaN fill: an element the launcher fails to write shows up as an error.
    void poison() {
        std::vector<float> h(n, NAN);
        put(h);
    }
};

std::vector<float> normal(uint64_t seed, size_t n, float scale) {
    std::vector<float> v(n);
    oracle_fill_normal(seed, v.data(), n);
    for (float& x : v) x *= scale;
    return v;
}

// Largest |got - want| relative to max(1, max|want|); NaN anywhere -> +inf.
double rel_err(const std::vector<float>& got, const std::vector<float>& want) {
    double err = 0.0, big = 1.0;
    for (size_t i = 0; i < want.size(); ++i) {
        const double g = got[i], w = want[i];
        if (!std::isfinite(g) || !std::isfinite(w)) return INFINITY;
        err = std::fmax(err, std::fabs(g - w));
        big = std::fmax(big, std::fabs(w));
    }
    return err / big;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 5) {
        std::fprintf(stderr, "usage: %s B S E H\n", argv[0]);
        return 2;
    }
    const int B = std::atoi(argv[1]), S = std::atoi(argv[2]), E = std::atoi(argv[3]), H = std::atoi(argv[4]);
    if (B <= 0 || S <= 0 || E <= 0 || H <= 0 || E % H != 0) {
        std::fprintf(stderr, "bad shape B=%d S=%d E=%d H=%d\n", B, S, E, H);
        return 2;
    }
    const size_t T = (size_t)B * S;
    const float wscale = 1.0f / std::sqrt((float)E);

    // Host inputs: layer input, weights and biases as HipGPT lays them out
    // ([in][out] row-major), and the gradient arriving at the attention output.
    const std::vector<float> x = normal(1, T * E, 1.0f);
    const std::vector<float> wqkv = normal(2, (size_t)E * 3 * E, wscale), bqkv = normal(3, 3 * (size_t)E, 0.1f);
    const std::vector<float> wo = normal(4, (size_t)E * E, wscale), bo = normal(5, E, 0.1f);
    const std::vector<float> gattn = normal(6, T * E, 1.0f);

    Dev d_x(T * E), d_wqkv(wqkv.size()), d_bqkv(bqkv.size()), d_wo(wo.size()), d_bo(bo.size());
    Dev d_qkv(3 * T * E), d_attn(T * E), d_out(T * E), d_probs((size_t)B * H * S * S);
    Dev d_gattn(T * E), d_gqkv(3 * T * E);
    d_x.put(x);
    d_wqkv.put(wqkv);
    d_bqkv.put(bqkv);
    d_wo.put(wo);
    d_bo.put(bo);
    d_gattn.put(gattn);
    d_qkv.poison();
    d_attn.poison();
    d_out.poison();
    d_probs.poison();
    d_gqkv.poison();

    // TransformerLayer::self_attention_forward
    launch_matmul_add_bias(d_x.p, d_wqkv.p, d_bqkv.p, d_qkv.p, (int)T, E, 3 * E);
    launch_multihead_attention(d_qkv.p, d_attn.p, d_probs.p, B, S, E, H);
    launch_matmul_add_bias(d_attn.p, d_wo.p, d_bo.p, d_out.p, (int)T, E, E);
    // TransformerLayer::backward, attention step
    launch_multihead_attention_backward(d_gattn.p, d_qkv.p, d_probs.p, d_gqkv.p, B, S, E, H);
    HIP_OK(hipGetLastError());
    HIP_OK(hipDeviceSynchronize());

    const std::vector<float> qkv = d_qkv.get(), attn = d_attn.get(), out = d_out.get();
    const std::vector<float> probs = d_probs.get(), gqkv = d_gqkv.get();

    // Oracle, stage by stage on the GPU's own stage inputs, so each error is
    // that stage's alone.
    std::vector<float> w_qkv(3 * T * E), w_attn(T * E), w_probs(probs.size()), w_out(T * E), w_gqkv(3 * T * E);
    oracle_matmul_add_bias(x.data(), wqkv.data(), bqkv.data(), w_qkv.data(), (int)T, E, 3 * E);
    if (oracle_launch_multihead_attention(qkv.data(), w_attn.data(), w_probs.data(), B, S, E, H, 0, 8) != 0) return 2;
    oracle_matmul_add_bias(attn.data(), wo.data(), bo.data(), w_out.data(), (int)T, E, E);
    if (oracle_mha_backward(gattn.data(), qkv.data(), probs.data(), w_gqkv.data(), B, S, E, H) != 0) return 2;

    const double e_qkv = rel_err(qkv, w_qkv), e_attn = rel_err(attn, w_attn), e_probs = rel_err(probs, w_probs);
    const double e_out = rel_err(out, w_out), e_gqkv = rel_err(gqkv, w_gqkv);
    std::printf("layer_dropin B=%d S=%d E=%d H=%d: qkv %.2e attn %.2e probs %.2e out %.2e grad_qkv %.2e\n", B, S,
                E, H, e_qkv, e_attn, e_probs, e_out, e_gqkv);
    const double tol = 1e-4;
    const bool ok = e_qkv <= tol && e_attn <= tol && e_probs <= tol && e_out <= tol && e_gqkv <= tol;
    std::printf("%s\n", ok ? "PASS" : "FAIL");
    return ok ? 0 : 1;
}
