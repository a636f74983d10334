// dn.hip — the two mixers of the hybrid (qwen35) decode that the dense model
// does not have: the gated delta-net step and the QK-norm + RoPE of the gated
// full-attention layers.
//
// Delta-net step (plano_delta, resident_forward.rs:2252-2470, with the math of
// delta_net.rs:13-131 and shaders dn_gates / dn_conv / dn_l2_qk / delta_net /
// dn_norm), one launch per layer and token.  Value head h owns a D x D f32
// state S_h (row j = value dim j, contiguous over the key dim) and reads key
// head h % k_heads (the modulo GQA of delta_net.comp:75-85):
//
//   gates   g = a_h * softplus(alpha_h . hn + dt_h), beta = sigmoid(beta_h . hn),
//           hn = rmsnorm(x) * attn_norm (f32 rows, as dn_gates reads b_normed)
//   conv    c = SiLU(sum_t w[t] x_{pos-W+1+t}) over the last W conv inputs
//   L2      q <- q / sqrt(|q|^2 + eps), k <- k / sqrt(|k|^2 + eps)
//   rule    S <- e^g S;  S_j <- S_j + beta (v_j - S_j . k) k;  o_j = S_j . q / sqrt(D)
//   norm    y_j = o_j / sqrt(mean_j(o^2) + eps) * norm_w[j] * silu(z_j)
//
// The rows of a head are independent in the rule, so a head is split over
// D/32 workgroups of 32 rows (one pack block each, on one XCD): the state streams from
// 4 x more CUs than one workgroup per head would use.  Each workgroup
// recomputes the head's gates, q and k (a few KB, L2-resident), packs its 32
// y values without the head's RMS factor and leaves its share of sum(o^2);
// the consumer (the ssm_out matvec) sums the shares of each head and scales
// the pack's block scales by the factor while it stages the pack (the pack is
// linear in its scale and block sums), so no workgroup waits for another.
// The conv inputs live in a ring of W slots indexed by position, so the slot
// being written (pos % W) is never one being read: workgroups that share a
// key head need no ordering.
#include "dn_dev.h"
#include "lrs_internal.h"
#include "pack_dev.h"

namespace lrs {


template <int CTRL>
__device__ __forceinline__ float dn_dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
// sum over each aligned group of 8 lanes, in every lane of the group
__device__ __forceinline__ float sum8(float v) {
    v += dn_dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dn_dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dn_dpp<0x141>(v);  // row_half_mirror
    return v;
}
__device__ __forceinline__ float wave_sum(float v) { return dn_wave_sum(v); }

template <int D>
__global__ __launch_bounds__(256) void k_dn_step(DnArgs a) {
    constexpr uint32_t R = D / 32;    // workgroups per head (32 rows each)
    constexpr int PPL = D / 32;       // float4 pieces of a row per lane (8 lanes per row)
    // workgroup b runs on XCD b % 8: with v_heads % 8 == 0 the R workgroups of
    // a head get ids of one residue mod 8, so the head's gate rows are fetched
    // into one XCD's L2 once instead of once per workgroup
    uint32_t r, hh;
    if (a.v_heads % 8 == 0) {
        const uint32_t x = blockIdx.x & 7, sl = blockIdx.x >> 3;
        hh = x + 8 * (sl / R);
        r = sl % R;
    } else {
        hh = blockIdx.x / R;
        r = blockIdx.x % R;
    }
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63, wave = tid >> 6;
    const uint32_t rho = tid >> 3, lam = tid & 7;  // row of the lane group, lane in the group
    const uint32_t j = 32 * r + rho;
    const uint32_t kh = hh % a.k_heads;
    const uint32_t KD = a.k_heads * D, CD = 2 * KD + a.v_heads * D;
    __shared__ __attribute__((aligned(16))) float sq[D], sk[D];
    __shared__ float sv[32], so[32], red[3][4], gb[2];

    // state row j in flight first: lane lam holds pieces 8c + lam
    float4 st[PPL];
    float4 *srow = reinterpret_cast<float4 *>(a.state + ((size_t)hh * D + j) * D);
#pragma unroll
    for (int c = 0; c < PPL; c++) st[c] = srow[8 * c + lam];

    // causal conv + SiLU of q, k (key head kh) and this workgroup's v rows
    // (dn_conv.comp); the current input goes to ring slot pos % W, written
    // once per channel: q/k by workgroup 0 of value head kh, v by its owner.
    // Two channels per thread (2D + 32 <= 512); their loads, like the gate
    // rows' below, are issued before any of them is used.  All W ring slots
    // are loaded (none of these loads waits for the position); the position
    // then picks the W - 1 previous inputs among them (slot pos % W, which
    // another workgroup may be overwriting, is never picked).
    const uint32_t W = a.d_conv;
    const bool own_qk = r == 0 && hh < a.k_heads;
    constexpr int WM = 8;  // d_conv <= 8
    float xc[2], wt[2][WM], wa[2][WM];
    uint32_t chs[2];
#pragma unroll
    for (int u = 0; u < 2; u++) {
        const uint32_t c = tid + 256 * u;
        const uint32_t ch = c < D ? kh * D + c
                            : c < 2 * D ? KD + kh * D + (c - D)
                                        : 2 * KD + hh * D + 32 * r + (c - 2 * D);
        chs[u] = ch;
        if (c < 2 * D + 32) {
            xc[u] = a.qkv[ch];
#pragma unroll
            for (int t = 0; t < WM; t++) {
                if ((uint32_t)t < W) {
                    wt[u][t] = a.conv_w[(size_t)ch * W + t];
                    wa[u][t] = a.win[(size_t)t * CD + ch];
                }
            }
        }
    }
    // the read-out's gate z and norm weight of this workgroup's 32 rows, for
    // the pack at the end
    float zr = 0.f, nr = 0.f;
    if (tid < 32) {
        zr = a.z[(size_t)hh * D + 32 * r + tid];
        nr = a.norm_w[32 * r + tid];
    }
    const uint32_t pos = a.step[1];
    const uint32_t wslot = pos % W;
    // gate projections of hn = rmsnorm(x) * attn_norm (dn_gates.comp): every
    // load of a thread's elements is issued before the first product; with
    // a.gates the projection launch computed them (its spare workgroups)
    float2 gpre = make_float2(0.f, 0.f);
    if (a.gates) {
        if (tid == 0) gpre = a.gates[hh];
    } else {
        DnGateRegs g;
        dn_gate_load(g, a.x, a.attn_norm, a.alpha + (size_t)hh * a.n_embd,
                     a.beta + (size_t)hh * a.n_embd, a.n_embd, tid);
        dn_gate_reduce(g, a.n_embd, tid, red);
    }

    // conv + SiLU
    {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const uint32_t c = tid + 256 * u;
            if (c >= 2 * D + 32) continue;
            float acc = 0.f;
#pragma unroll
            for (int t = 0; t < WM; t++) {
                if ((uint32_t)t + 1 < W) {
                    // input pos - W + 1 + t, in ring slot (pos + 1 + t) % W
                    const uint32_t sl = (pos + 1 + t) % W;
                    float wn = wa[u][0];
#pragma unroll
                    for (int q = 1; q < WM; q++)
                        if ((uint32_t)q == sl) wn = wa[u][q];
                    acc += wn * wt[u][t];
                }
            }
            float wl = wt[u][0];
#pragma unroll
            for (int t = 1; t < WM; t++)
                if ((uint32_t)t == W - 1) wl = wt[u][t];
            acc += xc[u] * wl;
            const float v = acc / (1.0f + expf(-acc));
            if (c < D) sq[c] = v;
            else if (c < 2 * D) sk[c - D] = v;
            else sv[c - 2 * D] = v;
            if (c >= 2 * D || own_qk) a.win[(size_t)wslot * CD + chs[u]] = xc[u];
        }
    }
    __syncthreads();

    if (tid == 0) {
        const float2 d = a.gates ? gpre : dn_gate_final(red, a.a[hh], a.dt[hh], a.n_embd, a.eps);
        gb[0] = d.x;  // decay e^g
        gb[1] = d.y;  // beta
    }
    // L2 norms of q and k (dn_l2_qk.comp); 1/sqrt(D) of the read-out folded into q
    {
        float qq = 0.f, kk = 0.f;
        for (uint32_t c = tid; c < (uint32_t)D; c += 256) {
            qq += sq[c] * sq[c];
            kk += sk[c] * sk[c];
        }
        qq = wave_sum(qq);
        kk = wave_sum(kk);
        __syncthreads();  // red[] reuse after the gate reduction above
        if (lane == 0) {
            red[0][wave] = qq;
            red[1][wave] = kk;
        }
    }
    __syncthreads();
    const float qq = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
    const float kk = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
    const float qs = 1.0f / sqrtf(qq + a.eps) * (1.0f / sqrtf((float)D));
    const float ks = 1.0f / sqrtf(kk + a.eps);
    const float decay = gb[0], beta = gb[1];

    // delta rule on row j: 8 lanes per row
    float4 kr[PPL], qr[PPL];
#pragma unroll
    for (int c = 0; c < PPL; c++) {
        const float4 k4 = reinterpret_cast<const float4 *>(sk)[8 * c + lam];
        const float4 q4 = reinterpret_cast<const float4 *>(sq)[8 * c + lam];
        kr[c] = make_float4(k4.x * ks, k4.y * ks, k4.z * ks, k4.w * ks);
        qr[c] = make_float4(q4.x * qs, q4.y * qs, q4.z * qs, q4.w * qs);
    }
    float pred = 0.f;
#pragma unroll
    for (int c = 0; c < PPL; c++) {
        st[c].x *= decay;
        st[c].y *= decay;
        st[c].z *= decay;
        st[c].w *= decay;
        pred += (st[c].x * kr[c].x + st[c].y * kr[c].y) + (st[c].z * kr[c].z + st[c].w * kr[c].w);
    }
    pred = sum8(pred);
    const float delta = (sv[rho] - pred) * beta;
    float o = 0.f;
#pragma unroll
    for (int c = 0; c < PPL; c++) {
        st[c].x = fmaf(delta, kr[c].x, st[c].x);
        st[c].y = fmaf(delta, kr[c].y, st[c].y);
        st[c].z = fmaf(delta, kr[c].z, st[c].z);
        st[c].w = fmaf(delta, kr[c].w, st[c].w);
        o += (st[c].x * qr[c].x + st[c].y * qr[c].y) + (st[c].z * qr[c].z + st[c].w * qr[c].w);
        srow[8 * c + lam] = st[c];
    }
    o = sum8(o);
    if (lam == 0) so[rho] = o;
    __syncthreads();

    // pack of o * norm_w * silu(z) for the 32 rows (dn_norm.comp mode 1 without
    // the head's RMS factor) and this workgroup's share of sum(o^2)
    if (tid < 32) {
        const uint32_t jj = 32 * r + tid;
        const float ov = so[tid];
        const float y = ov * (nr * (zr / (1.0f + expf(-zr))));
        pack_half(y, (hh * D + jj) >> 5, a.out);
        float p = ov * ov;
#pragma unroll
        for (int off = 16; off >= 1; off >>= 1) p += __shfl_xor(p, off, 64);
        if (tid == 0) a.part[hh * R + r] = p;
    }
}

hipError_t launch_dn_step(const DnArgs &a, uint32_t d_state, hipStream_t s) {
    if (a.k_heads == 0 || a.v_heads % a.k_heads || a.d_conv == 0 || a.d_conv > 8 ||
        a.n_embd % 4 || a.n_embd > 8192)
        return hipErrorInvalidValue;
    switch (d_state) {
    case 64: hipLaunchKernelGGL(k_dn_step<64>, dim3(2 * a.v_heads), dim3(256), 0, s, a); break;
    case 128: hipLaunchKernelGGL(k_dn_step<128>, dim3(4 * a.v_heads), dim3(256), 0, s, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// QK-norm + RoPE of the gated full-attention layer (resident_forward.rs:
// 3885-3963: dn_norm mode 2 on Q heads 2*head_dim apart and on K, then
// rope.comp), one workgroup per head: q heads (query half of the Q rows) to
// the contiguous q buffer, k heads with their v rows to the f16 cache at pos
template <int HD>
__global__ __launch_bounds__(HD) void k_qk_prep(const float *__restrict__ qg, const float *__restrict__ kb,
                                                const float *__restrict__ vb,
                                                const float *__restrict__ q_norm,
                                                const float *__restrict__ k_norm,
                                                const float *__restrict__ freq,
                                                const uint32_t *__restrict__ step, float *__restrict__ q,
                                                _Float16 *__restrict__ kc, _Float16 *__restrict__ vc,
                                                uint32_t n_head, uint32_t ctx, uint32_t rope_dim,
                                                float eps) {
    __shared__ float red[HD / 64];
    const uint32_t h = blockIdx.x, d = threadIdx.x, lane = d & 63, wave = d >> 6;
    const bool isq = h < n_head;
    const uint32_t kh = h - n_head;
    const float x = isq ? qg[(size_t)h * 2 * HD + d] : kb[(size_t)kh * HD + d];
    const float ss = wave_sum(x * x);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < HD / 64; w++) tot += red[w];
    const float s = 1.0f / sqrtf(tot / (float)HD + eps);
    float y = (x * s) * (isq ? q_norm[d] : k_norm[d]);
    const uint32_t pos = step[1];
    const float yo = __shfl_xor(y, 1, 64);
    if (d < rope_dim) {
        const float th = (float)pos * freq[d >> 1];
        float sn, cs;
        sincosf(th, &sn, &cs);
        y = (d & 1) ? yo * sn + y * cs : y * cs - yo * sn;
    }
    if (isq) {
        q[(size_t)h * HD + d] = y;
    } else {
        const size_t o = ((size_t)kh * ctx + pos) * HD + d;
        kc[o] = (_Float16)y;
        vc[o] = (_Float16)vb[(size_t)kh * HD + d];
    }
}

hipError_t launch_qk_prep(const float *qg, const float *kb, const float *vb, const float *q_norm,
                          const float *k_norm, const float *freq, const uint32_t *step, float *q,
                          _Float16 *kc, _Float16 *vc, uint32_t n_head, uint32_t n_kv,
                          uint32_t head_dim, uint32_t ctx, uint32_t rope_dim, float eps,
                          hipStream_t s) {
    const dim3 g(n_head + n_kv);
    switch (head_dim) {
    case 64:
        hipLaunchKernelGGL(k_qk_prep<64>, g, dim3(64), 0, s, qg, kb, vb, q_norm, k_norm, freq, step, q,
                           kc, vc, n_head, ctx, rope_dim, eps);
        break;
    case 128:
        hipLaunchKernelGGL(k_qk_prep<128>, g, dim3(128), 0, s, qg, kb, vb, q_norm, k_norm, freq, step,
                           q, kc, vc, n_head, ctx, rope_dim, eps);
        break;
    case 256:
        hipLaunchKernelGGL(k_qk_prep<256>, g, dim3(256), 0, s, qg, kb, vb, q_norm, k_norm, freq, step,
                           q, kc, vc, n_head, ctx, rope_dim, eps);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace lrs

// ---------------------------------------------------------------------------
// Batched prompt blocks of the hybrid model: nb tokens at positions pos0..,
// the same formulas as the decode kernels above, with the projections done
// by the matrix-core GEMMs (plano_delta with n_tok > 1,
// resident_forward.rs:2252-2470: dn_gates / dn_conv / dn_l2_qk / delta_net /
// dn_norm take the token dimension).
// ---------------------------------------------------------------------------
namespace lrs {

// gates per (token, value head) from the normalised rows hn (dn_gates.comp):
// gb[t][h] = {e^g, beta}, g = a_h * softplus(alpha_h . hn + dt_h)
__global__ __launch_bounds__(256) void k_dn_gates_rows(const float *__restrict__ hn,
                                                       const float *__restrict__ alpha,
                                                       const float *__restrict__ beta,
                                                       const float *__restrict__ a,
                                                       const float *__restrict__ dt,
                                                       float2 *__restrict__ gb, uint32_t n_embd,
                                                       uint32_t v_heads) {
    __shared__ float red[2][4];
    const uint32_t hh = blockIdx.x, t = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *x = hn + (size_t)t * n_embd;
    const float *al = alpha + (size_t)hh * n_embd, *be = beta + (size_t)hh * n_embd;
    float pa = 0.f, pb = 0.f;
    for (uint32_t i = 4 * tid; i < n_embd; i += 1024) {
        const float4 xv = *reinterpret_cast<const float4 *>(x + i);
        const float4 av = *reinterpret_cast<const float4 *>(al + i);
        const float4 bv = *reinterpret_cast<const float4 *>(be + i);
        pa += (av.x * xv.x + av.y * xv.y) + (av.z * xv.z + av.w * xv.w);
        pb += (bv.x * xv.x + bv.y * xv.y) + (bv.z * xv.z + bv.w * xv.w);
    }
    pa = wave_sum(pa);
    pb = wave_sum(pb);
    if (lane == 0) {
        red[0][wave] = pa;
        red[1][wave] = pb;
    }
    __syncthreads();
    if (tid == 0) {
        const float sa = (red[0][0] + red[0][1]) + (red[0][2] + red[0][3]);
        const float sb = (red[1][0] + red[1][1]) + (red[1][2] + red[1][3]);
        const float zz = sa + dt[hh];
        const float sp = zz > 20.0f ? zz : log1pf(expf(zz));
        gb[(size_t)t * v_heads + hh] = make_float2(expf(a[hh] * sp), 1.0f / (1.0f + expf(-sb)));
    }
}

// causal conv + SiLU over the block (dn_conv.comp): thread (channel c, row t)
// sums tap j times the input at position pos0 + t - (W-1) + j; inputs before
// the block come from the position ring (position P in slot P % W)
__global__ __launch_bounds__(256) void k_dn_conv_rows(const float *__restrict__ cin,
                                                      const float *__restrict__ conv_w,
                                                      const float *__restrict__ win, float *__restrict__ cout,
                                                      uint32_t cd, uint32_t W, uint32_t pos0) {
    const uint32_t c = blockIdx.x * 256 + threadIdx.x, t = blockIdx.y;
    if (c >= cd) return;
    float acc = 0.f;
    for (uint32_t j = 0; j < W; j++) {
        const int i = (int)t - (int)(W - 1) + (int)j;  // block row of the input (< 0: before the block)
        const float x = i >= 0 ? cin[(size_t)i * cd + c] : win[(size_t)((pos0 + W + i) % W) * cd + c];
        acc += x * conv_w[(size_t)c * W + j];
    }
    cout[(size_t)t * cd + c] = acc / (1.0f + expf(-acc));
}

// the block's last min(W, nb) inputs go to the ring at their positions (after
// k_dn_conv_rows has read the ring)
__global__ __launch_bounds__(256) void k_dn_ring_rows(const float *__restrict__ cin, float *__restrict__ win,
                                                      uint32_t cd, uint32_t W, uint32_t nb, uint32_t pos0) {
    const uint32_t c = blockIdx.x * 256 + threadIdx.x, i = nb - 1 - blockIdx.y;
    if (c >= cd) return;
    win[(size_t)((pos0 + i) % W) * cd + c] = cin[(size_t)i * cd + c];
}

// L2 norm of each q / k head of each token in place (dn_l2_qk.comp)
__global__ __launch_bounds__(128) void k_dn_l2_rows(float *__restrict__ co, uint32_t cd,
                                                    uint32_t d, float eps) {
    __shared__ float red[2];
    const uint32_t h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
    float *x = co + (size_t)t * cd + (size_t)h * d;
    float ss = 0.f;
    for (uint32_t i = tid; i < d; i += blockDim.x) ss += x[i] * x[i];
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const float tot = blockDim.x > 64 ? red[0] + red[1] : red[0];
    const float s = 1.0f / sqrtf(tot + eps);
    for (uint32_t i = tid; i < d; i += blockDim.x) x[i] *= s;
}

// the delta rule over the block: the state of 32 rows of a head stays in
// registers across the nb tokens (delta_net.comp's n_tok loop).  The tokens'
// q and k rows, this workgroup's 32 v values and the gates go through LDS in
// chunks of DNB_T tokens; the next chunk's loads are in flight while the
// current chunk is processed.  o[t][h*D + j]
constexpr uint32_t DNB_T = 16;
template <int D>
__global__ __launch_bounds__(256) void k_dn_block(const float *__restrict__ co, const float2 *__restrict__ gb,
                                                  float *__restrict__ state, float *__restrict__ o,
                                                  uint32_t k_heads, uint32_t v_heads, uint32_t nb) {
    constexpr uint32_t R = D / 32;
    constexpr int PPL = D / 32;
    constexpr uint32_t NP = D / 2 + 9;                  // float4 pieces per token: q, k, 32 v, gates
    constexpr uint32_t TF = 4 * NP;                     // floats per token in LDS
    constexpr uint32_t PPT = (DNB_T * NP + 255) / 256;  // pieces per thread per chunk
    __shared__ __attribute__((aligned(16))) float buf[2][DNB_T * TF];
    const uint32_t r = blockIdx.x % R, hh = blockIdx.x / R, tid = threadIdx.x;
    const uint32_t rho = tid >> 3, lam = tid & 7, j = 32 * r + rho;
    const uint32_t kh = hh % k_heads, KD = k_heads * D, CD = 2 * KD + v_heads * D;
    const float qscale = 1.0f / sqrtf((float)D);
    float4 pre[PPT];
    auto fetch = [&](uint32_t c0) {
#pragma unroll
        for (uint32_t p = 0; p < PPT; p++) {
            const uint32_t i = tid + 256 * p, t = i / NP, w = i % NP;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (i < DNB_T * NP && c0 + t < nb) {
                const float *row = co + (size_t)(c0 + t) * CD;
                if (w < D / 4)
                    v = reinterpret_cast<const float4 *>(row + (size_t)kh * D)[w];
                else if (w < D / 2)
                    v = reinterpret_cast<const float4 *>(row + KD + (size_t)kh * D)[w - D / 4];
                else if (w < D / 2 + 8)
                    v = reinterpret_cast<const float4 *>(row + 2 * KD + (size_t)hh * D + 32 * r)[w - D / 2];
                else {
                    const float2 g = gb[(size_t)(c0 + t) * v_heads + hh];
                    v = make_float4(g.x, g.y, 0.f, 0.f);
                }
            }
            pre[p] = v;
        }
    };
    auto stash = [&](float *b) {
#pragma unroll
        for (uint32_t p = 0; p < PPT; p++) {
            const uint32_t i = tid + 256 * p;
            if (i < DNB_T * NP) reinterpret_cast<float4 *>(b)[i] = pre[p];
        }
    };
    float4 st[PPL];
    float4 *srow = reinterpret_cast<float4 *>(state + ((size_t)hh * D + j) * D);
#pragma unroll
    for (int c = 0; c < PPL; c++) st[c] = srow[8 * c + lam];
    fetch(0);
    stash(buf[0]);
    __syncthreads();
    uint32_t cur = 0;
    for (uint32_t c0 = 0; c0 < nb; c0 += DNB_T) {
        const bool more = c0 + DNB_T < nb;
        if (more) fetch(c0 + DNB_T);
        const uint32_t nt = min(DNB_T, nb - c0);
        for (uint32_t tt = 0; tt < nt; tt++) {
            const float *tk = buf[cur] + tt * TF;
            const float4 *q4 = reinterpret_cast<const float4 *>(tk);
            const float4 *k4 = reinterpret_cast<const float4 *>(tk + D);
            float4 kr[PPL], qr[PPL];
#pragma unroll
            for (int c = 0; c < PPL; c++) {
                kr[c] = k4[8 * c + lam];
                qr[c] = q4[8 * c + lam];
            }
            const float vj = tk[2 * D + rho];
            const float2 g = make_float2(tk[2 * D + 32], tk[2 * D + 33]);
            float pred = 0.f;
#pragma unroll
            for (int c = 0; c < PPL; c++) {
                st[c].x *= g.x;
                st[c].y *= g.x;
                st[c].z *= g.x;
                st[c].w *= g.x;
                pred += (st[c].x * kr[c].x + st[c].y * kr[c].y) + (st[c].z * kr[c].z + st[c].w * kr[c].w);
            }
            pred = sum8(pred);
            const float delta = (vj - pred) * g.y;
            float ov = 0.f;
#pragma unroll
            for (int c = 0; c < PPL; c++) {
                st[c].x = fmaf(delta, kr[c].x, st[c].x);
                st[c].y = fmaf(delta, kr[c].y, st[c].y);
                st[c].z = fmaf(delta, kr[c].z, st[c].z);
                st[c].w = fmaf(delta, kr[c].w, st[c].w);
                ov += (st[c].x * qr[c].x + st[c].y * qr[c].y) + (st[c].z * qr[c].z + st[c].w * qr[c].w);
            }
            ov = sum8(ov);
            if (lam == 0) o[(size_t)(c0 + tt) * v_heads * D + (size_t)hh * D + j] = ov * qscale;
        }
        if (more) stash(buf[cur ^ 1]);
        __syncthreads();
        cur ^= 1;
    }
#pragma unroll
    for (int c = 0; c < PPL; c++) srow[8 * c + lam] = st[c];
}

// gated RMSNorm per (token, head): y = o / sqrt(mean(o^2) + eps) * w * silu(z)
// (dn_norm.comp mode 1)
__global__ __launch_bounds__(128) void k_dn_gnorm_rows(const float *__restrict__ o, const float *__restrict__ z,
                                                       const float *__restrict__ nw, float *__restrict__ y,
                                                       uint32_t vd, uint32_t d, float eps) {
    __shared__ float red[2];
    const uint32_t h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
    const size_t base = (size_t)t * vd + (size_t)h * d;
    float ss = 0.f;
    for (uint32_t i = tid; i < d; i += blockDim.x) ss += o[base + i] * o[base + i];
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __syncthreads();
    const float tot = blockDim.x > 64 ? red[0] + red[1] : red[0];
    const float s = 1.0f / sqrtf(tot / (float)d + eps);
    for (uint32_t i = tid; i < d; i += blockDim.x) {
        const float zz = z[base + i];
        y[base + i] = (o[base + i] * s) * (nw[i] * (zz / (1.0f + expf(-zz))));
    }
}

// gated attention of a block: QK-norm + RoPE per (token, head) at position
// pos0 + t; q to q[t][h*HD], k / v into the cache
template <int HD>
__global__ __launch_bounds__(HD) void k_qk_prep_rows(const float *__restrict__ qg, const float *__restrict__ kb,
                                                     const float *__restrict__ vb,
                                                     const float *__restrict__ q_norm,
                                                     const float *__restrict__ k_norm,
                                                     const float *__restrict__ freq, float *__restrict__ q,
                                                     _Float16 *__restrict__ kc, _Float16 *__restrict__ vc,
                                                     uint32_t n_head, uint32_t n_kv, uint32_t ctx,
                                                     uint32_t rope_dim, float eps, uint32_t pos0) {
    __shared__ float red[HD / 64];
    const uint32_t h = blockIdx.x, t = blockIdx.y, d = threadIdx.x, lane = d & 63, wave = d >> 6;
    const bool isq = h < n_head;
    const uint32_t kh = h - n_head;
    const float x = isq ? qg[((size_t)t * n_head + h) * 2 * HD + d] : kb[((size_t)t * n_kv + kh) * HD + d];
    const float ss = wave_sum(x * x);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int w = 0; w < HD / 64; w++) tot += red[w];
    const float s = 1.0f / sqrtf(tot / (float)HD + eps);
    float y = (x * s) * (isq ? q_norm[d] : k_norm[d]);
    const uint32_t pos = pos0 + t;
    const float yo = __shfl_xor(y, 1, 64);
    if (d < rope_dim) {
        const float th = (float)pos * freq[d >> 1];
        float sn, cs;
        sincosf(th, &sn, &cs);
        y = (d & 1) ? yo * sn + y * cs : y * cs - yo * sn;
    }
    if (isq) {
        q[((size_t)t * n_head + h) * HD + d] = y;
    } else {
        const size_t o = ((size_t)kh * ctx + pos) * HD + d;
        kc[o] = (_Float16)y;
        vc[o] = (_Float16)vb[((size_t)t * n_kv + kh) * HD + d];
    }
}

// att *= sigmoid(gate), gate = second half of each head's Q rows (gate_quant.comp)
__global__ __launch_bounds__(256) void k_gate_rows(float *__restrict__ att, const float *__restrict__ qg,
                                                   uint32_t qd, uint32_t hd, size_t n) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const size_t t = i / qd;
    const uint32_t e = (uint32_t)(i % qd), h = e / hd, dd = e % hd;
    const float g = qg[t * 2 * qd + (size_t)h * 2 * hd + hd + dd];
    att[i] = att[i] * (1.0f / (1.0f + expf(-g)));
}

hipError_t launch_dn_prefill(const DnBlockArgs &a, hipStream_t s) {
    const uint32_t D = a.d_state, KD = a.k_heads * D, VD = a.v_heads * D, CD = 2 * KD + VD;
    if (a.nb == 0 || a.n_embd % 4 || a.d_conv == 0 || a.d_conv > 8 || (D != 64 && D != 128))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_dn_gates_rows, dim3(a.v_heads, a.nb), dim3(256), 0, s, a.hn, a.alpha, a.beta,
                       a.a, a.dt, a.gb, a.n_embd, a.v_heads);
    hipLaunchKernelGGL(k_dn_conv_rows, dim3((CD + 255) / 256, a.nb), dim3(256), 0, s, a.cin, a.conv_w,
                       a.win, a.cout, CD, a.d_conv, a.pos0);
    hipLaunchKernelGGL(k_dn_ring_rows, dim3((CD + 255) / 256, min(a.d_conv, a.nb)), dim3(256), 0, s, a.cin,
                       a.win, CD, a.d_conv, a.nb, a.pos0);
    hipLaunchKernelGGL(k_dn_l2_rows, dim3(2 * a.k_heads, a.nb), dim3(128), 0, s, a.cout, CD, D, a.eps);
    if (D == 128)
        hipLaunchKernelGGL(k_dn_block<128>, dim3(4 * a.v_heads), dim3(256), 0, s, a.cout, a.gb, a.state,
                           a.o, a.k_heads, a.v_heads, a.nb);
    else
        hipLaunchKernelGGL(k_dn_block<64>, dim3(2 * a.v_heads), dim3(256), 0, s, a.cout, a.gb, a.state,
                           a.o, a.k_heads, a.v_heads, a.nb);
    hipLaunchKernelGGL(k_dn_gnorm_rows, dim3(a.v_heads, a.nb), dim3(128), 0, s, a.o, a.z, a.norm_w,
                       a.y, VD, D, a.eps);
    return hipGetLastError();
}

hipError_t launch_qk_prep_rows(const float *qg, const float *kb, const float *vb, const float *q_norm,
                               const float *k_norm, const float *freq, float *q, _Float16 *kc,
                               _Float16 *vc, uint32_t nb, uint32_t pos0, uint32_t n_head,
                               uint32_t n_kv, uint32_t head_dim, uint32_t ctx, uint32_t rope_dim,
                               float eps, hipStream_t s) {
    const dim3 g(n_head + n_kv, nb);
    switch (head_dim) {
    case 64:
        hipLaunchKernelGGL(k_qk_prep_rows<64>, g, dim3(64), 0, s, qg, kb, vb, q_norm, k_norm, freq, q, kc,
                           vc, n_head, n_kv, ctx, rope_dim, eps, pos0);
        break;
    case 128:
        hipLaunchKernelGGL(k_qk_prep_rows<128>, g, dim3(128), 0, s, qg, kb, vb, q_norm, k_norm, freq, q,
                           kc, vc, n_head, n_kv, ctx, rope_dim, eps, pos0);
        break;
    case 256:
        hipLaunchKernelGGL(k_qk_prep_rows<256>, g, dim3(256), 0, s, qg, kb, vb, q_norm, k_norm, freq, q,
                           kc, vc, n_head, n_kv, ctx, rope_dim, eps, pos0);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gate_rows(float *att, const float *qg, uint32_t nb, uint32_t qd, uint32_t hd,
                            hipStream_t s) {
    const size_t n = (size_t)nb * qd;
    hipLaunchKernelGGL(k_gate_rows, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, att, qg, qd, hd, n);
    return hipGetLastError();
}

}  // namespace lrs
