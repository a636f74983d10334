// attention.hip — batch-1 causal GQA decode attention over the f16 KV cache,
// split-K ("flash decode"): partials per (split, KV head), then a combine.
//
// Math of attention.rs:76-166 (scores q.k * 1/sqrt(head_dim), softmax,
// weighted sum of V, query head h reads KV head h / (n_head / n_head_kv)),
// over the f16 cache the reference GPU path keeps (kv_pack.comp,
// attention_split.comp + attn_reduce.comp): every split keeps (max, sum,
// unnormalised accumulator) and the combine rescales them, which is the
// online-softmax identity, exact up to f32 rounding.
//
// Cache layout (per layer): [n_head_kv][ctx][head_dim] f16, so a split's K
// (and V) rows are one contiguous run.  Each workgroup copies its K and V run
// straight into LDS with global_load_lds_dwordx4 (one HBM round trip, no
// VGPR staging), then: scores with HD/8 lanes per position (each lane owns 8
// dims as one 128-bit LDS read, the rep query heads of the KV head held in
// registers), softmax per head, the V sum with 2 dims per lane, and the
// partial (m, l, acc) to global memory.  The
// partials are rescaled and summed by a second, one-workgroup-per-head kernel
// (on this multi-XCD part a per-workgroup "last one combines" handshake needs
// an L2 writeback + invalidate per workgroup, which costs more than a launch).
#include "lrs_internal.h"
#include "pack_dev.h"

namespace lrs {

struct AttnArgs {
    const float *q;          // [n_head * HD], RoPE applied
    const _Float16 *kc, *vc; // this layer's caches
    XPack out;               // pack of the [n_head * HD] output (o-projection input)
    float *part;             // [n_head][S][HD + 4] split partials (acc, m, l, pad)
    const uint32_t *step;    // [token, pos]: attends positions 0..pos
    uint32_t n_head, n_kv, ctx, S, chunk_max;
    float scale;
};

constexpr int ATT_THREADS = 256;
constexpr int ATT_WAVES = ATT_THREADS / 64;
constexpr int ATT_MAX_REP = 8;

typedef __attribute__((address_space(3))) void lds_void;

// copies `bytes` (multiple of 16) from global to LDS, 1 KB per wave
// instruction (each lane 16 B); lanes past the end are masked off
__device__ __forceinline__ void copy_to_lds(const uint8_t *__restrict__ g, uint8_t *lds,
                                            uint32_t bytes) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (uint32_t base = wave * 1024; base < bytes; base += ATT_WAVES * 1024) {
        const uint32_t off = base + lane * 16;
        if (off < bytes)
            __builtin_amdgcn_global_load_lds(g + off, (lds_void *)(lds + base), 16, 0, 0);
    }
}

template <int HD>
__global__ __launch_bounds__(ATT_THREADS) void k_attn(AttnArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ float m_s[ATT_MAX_REP], l_s[ATT_MAX_REP];
    constexpr int LPP = HD / 8;        // lanes per position in the score phase
    constexpr int PPW = 64 / LPP;      // positions per wave and step
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t kh = blockIdx.y, s = blockIdx.x;
    const uint32_t rep = a.n_head / a.n_kv, h0 = kh * rep;
    const uint32_t L = a.step[1] + 1;
    const uint32_t chunk = (L + a.S - 1) / a.S;
    const uint32_t p0 = min(s * chunk, L), p1 = min(p0 + chunk, L), n = p1 - p0;

    _Float16 *ks = reinterpret_cast<_Float16 *>(smem);            // [chunk_max][HD]
    _Float16 *vs = ks + (size_t)a.chunk_max * HD;                 // [chunk_max][HD]
    float *sc = reinterpret_cast<float *>(vs + (size_t)a.chunk_max * HD);  // [rep][chunk_max]
    float *red = sc + ATT_MAX_REP * a.chunk_max;                  // [WAVES][rep][HD]

    // K and V runs of this split straight into LDS
    const size_t row0 = (size_t)kh * a.ctx + p0;
    copy_to_lds(reinterpret_cast<const uint8_t *>(a.kc + row0 * HD), reinterpret_cast<uint8_t *>(ks),
                n * HD * 2);
    copy_to_lds(reinterpret_cast<const uint8_t *>(a.vc + row0 * HD), reinterpret_cast<uint8_t *>(vs),
                n * HD * 2);
    // this lane's 8 dims of every query head of the group
    const uint32_t sub = lane % LPP, pw = lane / LPP;
    float qr[ATT_MAX_REP][8];
#pragma unroll
    for (int r = 0; r < ATT_MAX_REP; r++) {
        if (r < (int)rep) {
            const float4 *qp = reinterpret_cast<const float4 *>(a.q + (size_t)(h0 + r) * HD + 8 * sub);
            const float4 x0 = qp[0], x1 = qp[1];
            qr[r][0] = x0.x; qr[r][1] = x0.y; qr[r][2] = x0.z; qr[r][3] = x0.w;
            qr[r][4] = x1.x; qr[r][5] = x1.y; qr[r][6] = x1.z; qr[r][7] = x1.w;
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    // scores: positions in steps of PPW per wave, LPP lanes per position
    for (uint32_t pb = wave * PPW; pb < n; pb += ATT_WAVES * PPW) {
        const uint32_t pp = pb + pw;
        float acc[ATT_MAX_REP];
#pragma unroll
        for (int r = 0; r < ATT_MAX_REP; r++) acc[r] = 0.f;
        if (pp < n) {
            const uint4 raw = *reinterpret_cast<const uint4 *>(ks + (size_t)pp * HD + 8 * sub);
            const _Float16 *kv = reinterpret_cast<const _Float16 *>(&raw);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float kf = (float)kv[e];
#pragma unroll
                for (int r = 0; r < ATT_MAX_REP; r++)
                    if (r < (int)rep) acc[r] = fmaf(qr[r][e], kf, acc[r]);
            }
        }
#pragma unroll
        for (int r = 0; r < ATT_MAX_REP; r++) {
            if (r < (int)rep) {
                float v = acc[r];
#pragma unroll
                for (int o = LPP / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
                if (sub == 0 && pp < n) sc[r * a.chunk_max + pp] = v * a.scale;
            }
        }
    }
    __syncthreads();

    // per head: max, exp, sum (one wavefront per head)
    for (uint32_t r = wave; r < rep; r += ATT_WAVES) {
        float m = -INFINITY;
        for (uint32_t pp = lane; pp < n; pp += 64) m = fmaxf(m, sc[r * a.chunk_max + pp]);
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        float l = 0.f;
        for (uint32_t pp = lane; pp < n; pp += 64) {
            const float e = expf(sc[r * a.chunk_max + pp] - m);
            sc[r * a.chunk_max + pp] = e;
            l += e;
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) l += __shfl_xor(l, o, 64);
        if (lane == 0) {
            m_s[r] = m;
            l_s[r] = l;
        }
    }
    __syncthreads();

    // V: wave w sums positions w, w+WAVES, ...; lane owns HD/64 dims
    constexpr int DPL = HD / 64;
    float acc[ATT_MAX_REP][DPL];
#pragma unroll
    for (int r = 0; r < ATT_MAX_REP; r++)
#pragma unroll
        for (int k = 0; k < DPL; k++) acc[r][k] = 0.f;
    for (uint32_t pp = wave; pp < n; pp += ATT_WAVES) {
        float v[DPL];
        const _Float16 *vr = vs + (size_t)pp * HD + DPL * lane;
#pragma unroll
        for (int k = 0; k < DPL; k++) v[k] = (float)vr[k];
#pragma unroll
        for (int r = 0; r < ATT_MAX_REP; r++) {
            if (r < (int)rep) {
                const float p = sc[r * a.chunk_max + pp];
#pragma unroll
                for (int k = 0; k < DPL; k++) acc[r][k] = fmaf(p, v[k], acc[r][k]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < ATT_MAX_REP; r++)
        if (r < (int)rep)
#pragma unroll
            for (int k = 0; k < DPL; k++) red[((size_t)wave * rep + r) * HD + DPL * lane + k] = acc[r][k];
    __syncthreads();
    for (uint32_t i = tid; i < rep * HD; i += ATT_THREADS) {
        const uint32_t r = i / HD, d = i % HD;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < ATT_WAVES; w++) v += red[((size_t)w * rep + r) * HD + d];
        float *pr = a.part + ((size_t)(h0 + r) * a.S + s) * (HD + 4);
        pr[d] = v;
        if (d == 0) {
            pr[HD] = m_s[r];
            pr[HD + 1] = l_s[r];
        }
    }

}

// combine of the split partials of one query head (attn_reduce.comp): one
// workgroup per head, the kernel boundary after k_attn makes every split's
// partial visible (no per-workgroup L2 writeback / invalidate)
template <int HD>
__global__ __launch_bounds__(HD) void k_attn_combine(AttnArgs a) {
    extern __shared__ float w[];  // [S] split weights
    __shared__ float red[HD / 64];
    __shared__ float Msh;
    const uint32_t h = blockIdx.x, d = threadIdx.x, lane = d & 63, wave = d >> 6;
    constexpr uint32_t PR = HD + 4;
    const float *pr = a.part + (size_t)h * a.S * PR;
    float M = -INFINITY;
    for (uint32_t t = d; t < a.S; t += HD) M = fmaxf(M, pr[(size_t)t * PR + HD]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
    if (lane == 0) red[wave] = M;
    __syncthreads();
    if (d == 0) {
        float mm = red[0];
        for (int i = 1; i < HD / 64; i++) mm = fmaxf(mm, red[i]);
        Msh = mm;
    }
    __syncthreads();
    M = Msh;
    float den = 0.f;
    for (uint32_t t = d; t < a.S; t += HD) {
        const float mt = pr[(size_t)t * PR + HD];
        const float wt = mt == -INFINITY ? 0.f : expf(mt - M);
        w[t] = wt;
        den = fmaf(wt, pr[(size_t)t * PR + HD + 1], den);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) den += __shfl_xor(den, o, 64);
    __syncthreads();
    if (lane == 0) red[wave] = den;
    __syncthreads();
    float tot = 0.f;
    for (int i = 0; i < HD / 64; i++) tot += red[i];
    // all S loads of this thread's column are independent
    float num0 = 0.f, num1 = 0.f, num2 = 0.f, num3 = 0.f;
    uint32_t t = 0;
    for (; t + 4 <= a.S; t += 4) {
        num0 = fmaf(w[t], pr[(size_t)t * PR + d], num0);
        num1 = fmaf(w[t + 1], pr[(size_t)(t + 1) * PR + d], num1);
        num2 = fmaf(w[t + 2], pr[(size_t)(t + 2) * PR + d], num2);
        num3 = fmaf(w[t + 3], pr[(size_t)(t + 3) * PR + d], num3);
    }
    for (; t < a.S; t++) num0 = fmaf(w[t], pr[(size_t)t * PR + d], num0);
    pack_half(((num0 + num1) + (num2 + num3)) / tot, (h * HD + d) >> 5, a.out);
}

size_t attn_lds_bytes(uint32_t head_dim, uint32_t chunk_max) {
    const size_t kv = 2 * (size_t)chunk_max * head_dim * sizeof(_Float16);
    return kv + sizeof(float) * ((size_t)ATT_MAX_REP * chunk_max + (size_t)ATT_WAVES * ATT_MAX_REP * head_dim);
}

// splits so that a split holds at most 128 positions at full context
uint32_t attn_splits(uint32_t ctx) {
    uint32_t S = (ctx + 127) / 128;
    if (S < 8) S = 8;
    if (S > ctx) S = ctx;
    return S;
}

hipError_t launch_attention(const float *q, const _Float16 *kc, const _Float16 *vc, XPack out,
                            float *part, const uint32_t *step, uint32_t n_head, uint32_t n_kv,
                            uint32_t head_dim, uint32_t ctx, uint32_t S, hipStream_t s) {
    AttnArgs a;
    a.q = q;
    a.kc = kc;
    a.vc = vc;
    a.out = out;
    a.part = part;
    a.step = step;
    a.n_head = n_head;
    a.n_kv = n_kv;
    a.ctx = ctx;
    a.S = S;
    a.chunk_max = (ctx + S - 1) / S;
    a.scale = 1.0f / sqrtf((float)head_dim);
    if (n_head / n_kv > (uint32_t)ATT_MAX_REP) return hipErrorInvalidValue;
    const size_t lds = attn_lds_bytes(head_dim, a.chunk_max);
    if (lds > 160 * 1024) return hipErrorInvalidValue;
    dim3 grid(S, n_kv);
    const size_t wl = S * sizeof(float);
    switch (head_dim) {
    case 64:
        hipLaunchKernelGGL(k_attn<64>, grid, dim3(ATT_THREADS), lds, s, a);
        hipLaunchKernelGGL(k_attn_combine<64>, dim3(n_head), dim3(64), wl, s, a);
        break;
    case 128:
        hipLaunchKernelGGL(k_attn<128>, grid, dim3(ATT_THREADS), lds, s, a);
        hipLaunchKernelGGL(k_attn_combine<128>, dim3(n_head), dim3(128), wl, s, a);
        break;
    case 256:
        hipLaunchKernelGGL(k_attn<256>, grid, dim3(ATT_THREADS), lds, s, a);
        hipLaunchKernelGGL(k_attn_combine<256>, dim3(n_head), dim3(256), wl, s, a);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace lrs
