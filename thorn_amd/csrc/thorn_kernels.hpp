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

// Magma statistics (thorn.py:806-836): sums of g*m, g*g and m*m, where m is the moment before this
// step's update.
struct MagmaSums {
    float gm = 0.f, gg = 0.f, mm = 0.f;
    __device__ __forceinline__ void add(float g, float m) {
        gm = fmaf(g, m, gm);
        gg = fmaf(g, g, gg);
        mm = fmaf(m, m, mm);
    }
    __device__ __forceinline__ void add(const float4& part) {
        gm += part.x;
        gg += part.y;
        mm += part.z;
    }
};

// Block reduction of MagmaSums in a fixed order; every thread returns the totals. `scratch` holds
// at least 3 * blockDim.x / 64 floats.
__device__ __forceinline__ MagmaSums block_sum(MagmaSums v, float* scratch) {
    v.gm = wave_sum(v.gm);
    v.gg = wave_sum(v.gg);
    v.mm = wave_sum(v.mm);
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) {
        scratch[3 * wid] = v.gm;
        scratch[3 * wid + 1] = v.gg;
        scratch[3 * wid + 2] = v.mm;
    }
    __syncthreads();
    MagmaSums t;
    for (int i = 0; i < nw; ++i) t.add(make_float4(scratch[3 * i], scratch[3 * i + 1], scratch[3 * i + 2], 0.f));
    return t;
}

// s <- p s + (1 - p) sigmoid(cos / tau) with p = 0.9, tau = 2 (thorn.py:806-830); cos as
// torch.nn.functional.cosine_similarity computes it, each norm clamped at eps = 1e-8. The constants
// are the fp32 roundings of the reference's Python scalars, as its fp32 tensor ops use them.
__device__ __forceinline__ void magma_update(const MagmaSums& t, float* s) {
    const float gn = fmaxf(sqrtf(t.gg), 1e-8f), mn = fmaxf(sqrtf(t.mm), 1e-8f);
    const float cs = t.gm / (gn * mn);
    const float st = sigmoid_f(cs / 2.f);
    const float s_old = ldg<float>(s);
    stg<float>(s, 0.9f * s_old + 0.1f * st);
}

}  // namespace thorn
