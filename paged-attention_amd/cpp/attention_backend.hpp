#pragma once
// The reference's abstract single-query attention backend
// (include/attention_backend.hpp:3-8), unchanged: callers written against it
// keep compiling.

class AttentionBackend {
public:
    virtual void run(const float* q, const float* K, const float* V, float* out, int T, int d) = 0;
    virtual const char* name() const = 0;
    virtual ~AttentionBackend() = default;
};
