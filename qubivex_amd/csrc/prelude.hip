// The attention prelude that feeds the append: bias, clip, Q/K RMSNorm (full width or per
// head), RoPE.  Bit-exact with the reference's host forward pass
// (crates/qubivex-arch/src/lib.rs:1258-1292), whose arithmetic is plain f32 with explicit
// fused multiply-adds only in the norm's sum of squares:
//   bias:   y += b                                             (lib.rs:1259-1265)
//   clip:   z.clamp(-c, c)                                     (lib.rs:1266-1272)
//   norm:   x = (x * r) * w,  r = 1 / sqrt(ss / n + eps)       (math.rs:89-116)
//           ss = the 64-lane fma shape of reduce::dot (reduce.rs:1-50): lane l sums
//           x[i]^2 for i = l, l+64, ... in order; then a[i] += a[i+w] for w = 32..4;
//           then (a0 + a1) + (a2 + a3)
//   rope:   y1 = x1*c - x2*s,  y2 = x2*c + x1*s  (pairs i, i + d/2; math.rs:160-169)
// One wave per (token, part), its 64 lanes being the reduction's 64 lanes.  Floating-
// point contraction is off in this file: every product and sum rounds on its own.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "internal.h"

#pragma clang fp contract(off)

namespace qvkv {

// reduce::reduce of the 64 per-lane partial sums (every lane returns the total).
__device__ __forceinline__ float lane_tree(float a) {
#pragma unroll
    for (int w = 32; w >= 4; w >>= 1) a = a + __shfl_down(a, w);
    const float a1 = __shfl(a, 1), a2 = __shfl(a, 2), a3 = __shfl(a, 3);
    const float t = (__shfl(a, 0) + a1) + (a2 + a3);
    return t;
}

// rms_scale_of: correctly rounded division and square root, in this order.
__device__ __forceinline__ float rms_scale_of(float ss, float n, float eps) {
    return 1.0f / sqrtf(ss / n + eps);
}

__global__ __launch_bounds__(64) void k_prelude(float *__restrict__ q, float *__restrict__ k,
                                                float *__restrict__ v, uint32_t heads,
                                                uint32_t kvh, uint32_t d, PreludeArgs a) {
    extern __shared__ float xs[];
    const uint32_t t = blockIdx.x / 3, part = blockIdx.x % 3, lane = threadIdx.x;
    const uint32_t n = part == 0 ? heads * d : kvh * d;
    float *x = (part == 0 ? q : part == 1 ? k : v) + (uint64_t)t * n;
    const float *bias = part == 0 ? a.q_bias : part == 1 ? a.k_bias : a.v_bias;
    for (uint32_t i = lane; i < n; i += 64) {
        float z = x[i];
        if (bias) z = z + bias[i];
        if (a.has_clip) z = z < -a.clip ? -a.clip : (z > a.clip ? a.clip : z);
        xs[i] = z;
    }
    __syncthreads();
    if (part == 2) {  // values: bias and clip only
        for (uint32_t i = lane; i < n; i += 64) x[i] = xs[i];
        return;
    }
    const float *w = part == 0 ? a.q_norm : a.k_norm;
    if (a.norm == QVKV_NORM_FULL && w) {
        float acc = 0.0f;
        for (uint32_t i = lane; i < n; i += 64) acc = fmaf(xs[i], xs[i], acc);
        const float r = rms_scale_of(lane_tree(acc), (float)n, a.eps);
        __syncthreads();
        for (uint32_t i = lane; i < n; i += 64) xs[i] = (xs[i] * r) * w[i];
    } else if (a.norm == QVKV_NORM_PER_HEAD && w) {
        for (uint32_t hd = 0; hd < n / d; hd++) {
            float *h = xs + hd * d;
            float acc = 0.0f;
            for (uint32_t i = lane; i < d; i += 64) acc = fmaf(h[i], h[i], acc);
            const float r = rms_scale_of(lane_tree(acc), (float)d, a.eps);
            __syncthreads();
            for (uint32_t i = lane; i < d; i += 64) h[i] = (h[i] * r) * w[i];
            __syncthreads();
        }
    }
    __syncthreads();
    const uint32_t half = d / 2;
    const float *cs = a.rope + (uint64_t)t * d;
    for (uint32_t u = lane; u < (n / d) * half; u += 64) {
        const uint32_t hd = u / half, i = u - hd * half;
        const float x1 = xs[hd * d + i], x2 = xs[hd * d + i + half];
        const float c = cs[i], s = cs[half + i];
        const float p1 = x1 * c, p2 = x2 * s, p3 = x2 * c, p4 = x1 * s;
        x[hd * d + i] = p1 - p2;
        x[hd * d + i + half] = p3 + p4;
    }
}

hipError_t launch_prelude(float *q, float *k, float *v, uint32_t s, uint32_t heads,
                          uint32_t kvh, uint32_t d, const PreludeArgs &a, hipStream_t st) {
    if (s == 0) return hipSuccess;
    const uint64_t lds = (uint64_t)(heads > kvh ? heads : kvh) * d * 4;
    hipLaunchKernelGGL(k_prelude, dim3(s * 3), dim3(64), (uint32_t)lds, st, q, k, v, heads, kvh,
                       d, a);
    return hipGetLastError();
}

}  // namespace qvkv
