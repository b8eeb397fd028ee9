// Elementwise update math shared by the THORN kernels. The library is compiled with
// -ffp-contract=off, so every multiply and add below rounds separately, as PyTorch's eager CPU
// ops do; explicit fmaf marks the places where PyTorch's vectorized kernels fuse
// (add with alpha, lerp).
#pragma once

#include "thorn_common.hpp"

namespace thorn {

// Cautious weight decay and write-back (thorn.py:669-681, 702):
//   mask = (u * p >= 0); u += p * (mask * wd); p -= lr * u
__device__ __forceinline__ float cautious_step(float p, float u, float lr, float wd) {
    if (wd > 0.f) {
        const float mask = (u * p >= 0.f) ? wd : 0.f;
        u = u + p * mask;
    }
    return fmaf(u, -lr, p);
}

// torch.lerp(start, end, w) as ATen's vectorized CPU kernel computes it.
__device__ __forceinline__ float lerp_torch(float start, float end, float w) {
    const float diff = end - start;
    return fabsf(w) < 0.5f ? fmaf(w, diff, start) : fmaf(w - 1.f, diff, end);
}

// w1 = 1 - beta1 and w2 = 1 - beta2 are computed in double on the host and rounded once, as the
// reference's Python scalars are before they reach the fp32 tensor ops.
struct AdamScalars {
    float lr, wd, beta2, w1, w2, bc1, bc2, eps;
    bool apply, degenerate, atan2_mode;
};

// Adam / Adam-atan2 element update (thorn.py:876-888): m and v always move; p only when applied.
__device__ __forceinline__ void adam_elem(float& p, float g, float& m, float& v, const AdamScalars& s) {
    m = lerp_torch(m, g, s.w1);
    v = v * s.beta2 + s.w2 * g * g;
    if (!s.apply) return;
    float u;
    if (s.degenerate) {
        u = m;
    } else if (s.atan2_mode) {
        u = atan2f(m * s.bc1, sqrtf(v * s.bc2));
    } else {
        u = (m * s.bc1) / (sqrtf(v * s.bc2) + s.eps);
    }
    p = cautious_step(p, u, s.lr, s.wd);
}

}  // namespace thorn
