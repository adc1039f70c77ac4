#pragma once
// The legacy interface's CPU backend (src/attention/cpu/attention.hpp:5-11):
// single-query, single-head fp32 attention on the host. It is a backend of its
// own behind AttentionBackend, as in the reference; no GPU entry point of this
// library calls it.

#include "attention_backend.hpp"

#include <algorithm>
#include <cmath>
#include <vector>

// out[d] = sum_t softmax_t(q . K[t] / sqrt(d)) V[t], K and V row-major [T][d],
// all fp32 in the order of src/attention/cpu/attention.cpp:14-34: scaled dot
// products, the running maximum, exp of the shifted scores, their sum, then the
// weighted sum of V rows divided by it.
inline void cpu_attention(const float* q, const float* K, const float* V, float* out, int T, int d) {
    std::vector<float> w(static_cast<size_t>(T));
    const float scale = 1.0f / std::sqrt(static_cast<float>(d));
    float mx = -INFINITY;
    for (int t = 0; t < T; ++t) {
        float s = 0.0f;
        for (int i = 0; i < d; ++i) s += q[i] * K[static_cast<size_t>(t) * d + i];
        w[static_cast<size_t>(t)] = s * scale;
        mx = std::max(mx, w[static_cast<size_t>(t)]);
    }
    float sum = 0.0f;
    for (int t = 0; t < T; ++t) {
        w[static_cast<size_t>(t)] = std::exp(w[static_cast<size_t>(t)] - mx);
        sum += w[static_cast<size_t>(t)];
    }
    for (int t = 0; t < T; ++t) w[static_cast<size_t>(t)] /= sum;
    for (int i = 0; i < d; ++i) {
        float acc = 0.0f;
        for (int t = 0; t < T; ++t) acc += w[static_cast<size_t>(t)] * V[static_cast<size_t>(t) * d + i];
        out[i] = acc;
    }
}

class CpuAttention : public AttentionBackend {
public:
    void run(const float* q, const float* K, const float* V, float* out, int T, int d) override {
        cpu_attention(q, K, V, out, T, d);
    }
    const char* name() const override { return "cpu"; }
};
