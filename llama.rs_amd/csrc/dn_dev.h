// Device helpers of the delta net's gate projections (dn_gates.comp):
// g = a_h * softplus(alpha_h . hn + dt_h), beta = sigmoid(beta_h . hn),
// hn = rmsnorm(x) * attn_norm.  Shared by the step kernel (dn.hip), which
// computes them itself, and the delta-net projection launch (mq.hip), whose
// spare workgroups compute them for the step.  256 threads take a head's
// dots: thread t holds the float4 groups 4t + 1024 g (n_embd <= 8192).
#pragma once

#include "lrs_internal.h"

namespace lrs {

constexpr int DN_GATE_THREADS = 256;

// the gate projections of every value head, for the projection launch's
// spare workgroups (launch_mq with gates): out[h] = {e^g, beta} of head h
struct DnGateArgs {
    const float *x, *attn_norm;   // residual [n_embd], its norm weight
    const float *alpha, *beta;    // [v_heads][n_embd]
    const float *a, *dt;          // [v_heads]
    float2 *out;                  // [v_heads]
    uint32_t n_embd, v_heads;
    float eps;
};
constexpr int DN_GI = 8;  // float4 per thread per row: n_embd <= 8192

struct DnGateRegs {
    float4 xv[DN_GI], wv[DN_GI], av[DN_GI], bv[DN_GI];
};

// the gate projections' operands of thread tid (< 256): every load is
// issued before the first product
__device__ __forceinline__ void dn_gate_load(DnGateRegs &g, const float *__restrict__ x,
                                             const float *__restrict__ nw,
                                             const float *__restrict__ al,
                                             const float *__restrict__ be, uint32_t n_embd,
                                             uint32_t tid) {
#pragma unroll
    for (int k = 0; k < DN_GI; k++) {
        const uint32_t i = 4 * tid + 1024 * k;
        if (i < n_embd) {
            g.xv[k] = *reinterpret_cast<const float4 *>(x + i);
            g.wv[k] = *reinterpret_cast<const float4 *>(nw + i);
            g.av[k] = *reinterpret_cast<const float4 *>(al + i);
            g.bv[k] = *reinterpret_cast<const float4 *>(be + i);
        }
    }
}

__device__ __forceinline__ float dn_wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// one float4 group into a thread's running sums of x^2, alpha . hn, beta . hn
__device__ __forceinline__ void dn_gate_accum(float4 xq, float4 wq, float4 aq, float4 bq, float &ss,
                                              float &pa, float &pb) {
    ss += (xq.x * xq.x + xq.y * xq.y) + (xq.z * xq.z + xq.w * xq.w);
    const float h0 = xq.x * wq.x, h1 = xq.y * wq.y, h2 = xq.z * wq.z, h3 = xq.w * wq.w;
    pa += (aq.x * h0 + aq.y * h1) + (aq.z * h2 + aq.w * h3);
    pb += (bq.x * h0 + bq.y * h1) + (bq.z * h2 + bq.w * h3);
}

// the running sums over the wavefront; lane 0 of wavefront w (< 4) writes
// red[0..2][w]
__device__ __forceinline__ void dn_gate_store(float ss, float pa, float pb, uint32_t tid,
                                              float (*red)[4]) {
    ss = dn_wave_sum(ss);
    pa = dn_wave_sum(pa);
    pb = dn_wave_sum(pb);
    if ((tid & 63) == 0) {
        red[0][tid >> 6] = ss;
        red[1][tid >> 6] = pa;
        red[2][tid >> 6] = pb;
    }
}

// thread tid's sums over its groups (in group order), then dn_gate_store
__device__ __forceinline__ void dn_gate_reduce(const DnGateRegs &g, uint32_t n_embd, uint32_t tid,
                                               float (*red)[4]) {
    float ss = 0.f, pa = 0.f, pb = 0.f;
#pragma unroll
    for (int k = 0; k < DN_GI; k++)
        if (4 * tid + 1024 * k < n_embd) dn_gate_accum(g.xv[k], g.wv[k], g.av[k], g.bv[k], ss, pa, pb);
    dn_gate_store(ss, pa, pb, tid, red);
}

// the same sums with the loads in two rounds of half the groups (half the
// registers; the same order of additions, so the same result)
__device__ __forceinline__ void dn_gate_two_rounds(const float *__restrict__ x,
                                                   const float *__restrict__ nw,
                                                   const float *__restrict__ al,
                                                   const float *__restrict__ be, uint32_t n_embd,
                                                   uint32_t tid, float (*red)[4]) {
    constexpr int H = DN_GI / 2;
    float ss = 0.f, pa = 0.f, pb = 0.f;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        float4 xv[H], wv[H], av[H], bv[H];
#pragma unroll
        for (int k = 0; k < H; k++) {
            const uint32_t i = 4 * tid + 1024 * (H * h + k);
            if (i < n_embd) {
                xv[k] = *reinterpret_cast<const float4 *>(x + i);
                wv[k] = *reinterpret_cast<const float4 *>(nw + i);
                av[k] = *reinterpret_cast<const float4 *>(al + i);
                bv[k] = *reinterpret_cast<const float4 *>(be + i);
            }
        }
#pragma unroll
        for (int k = 0; k < H; k++)
            if (4 * tid + 1024 * (H * h + k) < n_embd) dn_gate_accum(xv[k], wv[k], av[k], bv[k], ss, pa, pb);
    }
    dn_gate_store(ss, pa, pb, tid, red);
}

// {decay e^g, beta} from the four wavefronts' sums (delta_net.rs:13-20)
__device__ __forceinline__ float2 dn_gate_final(const float (*red)[4], float a_h, float dt_h,
                                                uint32_t n_embd, float eps) {
    const float ss = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
    const float pa = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
    const float pb = (red[2][0] + red[2][1]) + (red[2][2] + red[2][3]);
    const float s = 1.0f / sqrtf(ss / (float)n_embd + eps);
    const float zz = pa * s + dt_h;
    const float sp = zz > 20.0f ? zz : log1pf(expf(zz));
    return make_float2(expf(a_h * sp), 1.0f / (1.0f + expf(-(pb * s))));
}

}  // namespace lrs
