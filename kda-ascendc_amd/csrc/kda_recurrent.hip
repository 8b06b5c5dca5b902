// Token-by-token KDA recurrence in fp32: the decode step (T = 1) and the
// fused-recurrent form of the forward for any T.
//
// Per value head and token t, with S the [V, K] fp32 state:
//   S     = S * alpha_t[None, :]
//   v_new = beta_t * (v_t - S k^_t)
//   S     = S + v_new k^_t^T
//   o_t   = scale * S q^_t
// alpha_t = exp(lb * sigmoid(exp(A_log) * (g_t + dt_bias))) with the in-kernel
// gate; else exp(g_t) when g is the per-token log decay (g_log), else
// 2^(G_t - G_{t-1}) with G the chunk-local log2 cumsum the chunked path takes
// (G_{-1} = 0 at every 16-token chunk start of a sequence).  This is the recurrence the
// chunked path is the WY form of (kernels.py:53-302 computes it chunk-wise);
// the reference's tests use FLA's fused_recurrent_kda for it
// (/root/reference/tests/test_kda_bt16.py:26-38), and its roadmap lists the
// decode step (README.md:503-505).  No rounding happens between tokens, so
// with o in fp32 the kernel is also an on-GPU gold for the chunked path.
//
// One work-group of 256 threads per (sequence or batch row, value head).
// Thread t = 32 * hw + j holds the 64 state elements at memory offsets
// 1024 * i + 4 * t + c (i = 0..15, c = 0..3) of the head's 128 x 128 state,
// so every state load and store is a 16-byte access and each wave
// instruction covers 1 KiB of consecutive memory, in either layout.  What
// those elements are depends on the layout:
//   V-first ([V, K], row v contiguous): S[v = 8i + hw][k = 4j + c].  The
//     products S k^ and S q^ reduce over k across the 32 lanes of a
//     half-wave (hw), which all hold one set of rows.
//   K-first ([K, V]): S[v = 4j + c][k = 8i + hw].  The products reduce
//     over i in registers, then over the eight half-waves: lane pairs of a
//     wave by a shuffle, the four waves through LDS.
// The state lives in registers for the whole sequence (64 floats per
// thread, 165 VGPRs in all), so three work-groups share a CU and the decode
// step streams the states at close to the memory system's rate.
// Grouped value heads (GVA): value head hv reads q/k head hv / (HV / H)
// (kernels.py:88).  Varlen: one work-group per (sequence, value head), over
// the sequence's tokens, with states [N, HV, ...].
#include "kda_common.h"

namespace kda {

namespace {

constexpr int RT = 256;  // threads per work-group

__device__ __forceinline__ float load_scalar(const void* base, int is_bf16, int64_t i) {
    return is_bf16 ? bf2f(static_cast<const uint16_t*>(base)[i])
                   : static_cast<const float*>(base)[i];
}

// Sum over the 32 lanes of a half-wave; every lane receives it: each 16-lane
// row by DPP, then the two rows by one swizzle.  Every lane adds the same
// operands in the same order, so all receive the same bits.
__device__ __forceinline__ float half_sum(float x) {
    x = row_sum16(x);
    return x + xor16(x);
}

__device__ __forceinline__ float sigmoid_precise(float x) { return 1.0f / (1.0f + expf(-x)); }

// The decay alpha of one element of a token, in the three gate modes; gp is
// the element's G_{t-1} of the cumsum form (reset every 16 tokens).
__device__ __forceinline__ float decay_of(const Params& p, float g, float ea, float dtb, float& gp,
                                          bool chunk_start) {
    if (p.use_gate) return expf(p.lower_bound * sigmoid_precise(ea * (g + dtb)));
    if (p.g_log) return expf(g);
    if (chunk_start) gp = 0.0f;
    const float a = exp2f(g - gp);
    gp = g;
    return a;
}

// One token's raw inputs for this thread.  V-first: q, k and g at the
// thread's columns 4j .. 4j+3 and, for threads 0..31, v[4t .. 4t+3] (staged
// for the work-group).  K-first: q, k and g at columns 2l, 2l+1 for the
// lanes l of wave 0 (which form the token's vectors), and v[4j .. 4j+3]
// for every thread.  beta for all.
struct TokRaw {
    u32x2 q, k;
    float g[4];
    float beta;
    u32x2 v;
};

template <bool VFIRST>
__device__ __forceinline__ void load_tok(const Params& p, const SeqSpan& sp, int tt, int h, int hv,
                                         int t, TokRaw& r) {
    const int64_t rq = (sp.tok0 + tt) * p.H + h;
    const int64_t rv = (sp.tok0 + tt) * p.HV + hv;
    const int j = t & 31;
    r.q = r.k = r.v = u32x2{0u, 0u};
#pragma unroll
    for (int c = 0; c < 4; ++c) r.g[c] = 0.f;
    if (VFIRST) {
        const int col = 4 * j;
        r.q = *reinterpret_cast<const u32x2*>(p.q + rq * DK + col);
        r.k = *reinterpret_cast<const u32x2*>(p.k + rq * DK + col);
        if (p.g_bf16) {
            const u32x2 gw =
                *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(p.g) + rv * DK + col);
            r.g[0] = __builtin_bit_cast(float, gw.x << 16);
            r.g[1] = __builtin_bit_cast(float, gw.x & 0xffff0000u);
            r.g[2] = __builtin_bit_cast(float, gw.y << 16);
            r.g[3] = __builtin_bit_cast(float, gw.y & 0xffff0000u);
        } else {
            const f32x4 gv =
                *reinterpret_cast<const f32x4*>(static_cast<const float*>(p.g) + rv * DK + col);
#pragma unroll
            for (int c = 0; c < 4; ++c) r.g[c] = gv[c];
        }
        if (t < 32) r.v = *reinterpret_cast<const u32x2*>(p.v + rv * DK + 4 * t);
    } else {
        if (t < 64) {
            const int col = 2 * t;
            r.q.x = *reinterpret_cast<const uint32_t*>(p.q + rq * DK + col);
            r.k.x = *reinterpret_cast<const uint32_t*>(p.k + rq * DK + col);
            if (p.g_bf16) {
                const uint32_t gw =
                    *reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(p.g) + rv * DK + col);
                r.g[0] = __builtin_bit_cast(float, gw << 16);
                r.g[1] = __builtin_bit_cast(float, gw & 0xffff0000u);
            } else {
                const f32x2 gv =
                    *reinterpret_cast<const f32x2*>(static_cast<const float*>(p.g) + rv * DK + col);
                r.g[0] = gv.x;
                r.g[1] = gv.y;
            }
        }
        r.v = *reinterpret_cast<const u32x2*>(p.v + rv * DK + 4 * j);
    }
    r.beta = load_scalar(p.beta, p.beta_bf16, rv);
}

__device__ __forceinline__ float lo16(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float hi16(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

__device__ __forceinline__ void store_o(const Params& p, int64_t idx, float x) {
    if (p.o_fp32) {
        reinterpret_cast<float*>(p.o)[idx] = x;
    } else {
        p.o[idx] = f2bf(x);
    }
}

// ONE: a fixed-length batch of single tokens (the decode step): no token
// loop and no next-token prefetch, which leaves room for four waves per
// SIMD, so the 4 x 256 work-groups a CU holds stream the states in whole
// rounds.
template <bool VFIRST, bool ONE>
__global__ __launch_bounds__(RT) __attribute__((amdgpu_waves_per_eu(ONE ? 4 : 1))) void recurrent_kernel(Params p) {
    const int HV = p.HV, H = p.H;
    const int bhv = blockIdx.x;  // (batch row or sequence) * HV + hv
    const int hv = bhv - (bhv / HV) * HV;
    const int h = hv / (HV / H);
    const SeqSpan sp = seq_span(p, bhv);
    const int t = threadIdx.x;
    const int w = t >> 6, hw = t >> 5, j = t & 31;
    const int64_t sbase = (int64_t)bhv * DK * DK;

    // V-first: the token's v, double-buffered by token parity.
    __shared__ __attribute__((aligned(16))) float s_v[2][DK];
    // K-first: the token's decay, k^ and q^ (formed by wave 0), and the
    // per-wave partial sums of S k^ and S q^.
    __shared__ __attribute__((aligned(16))) float s_vec[3][DK];
    __shared__ __attribute__((aligned(16))) float s_red[2][4][DK];

    f32x4 S[16];
    const float* h0 = p.h0 ? p.h0 + sbase : nullptr;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        S[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (h0) S[i] = *reinterpret_cast<const f32x4*>(h0 + 1024 * i + 4 * t);
    }

    const float ea = p.use_gate ? expf(p.A_log[hv]) : 0.0f;
    // V-first: every thread forms its columns 4j .. 4j+3; K-first: wave 0
    // forms columns 2*lane, 2*lane+1 for the work-group.
    const int col = VFIRST ? 4 * j : 2 * (t & 63);
    const bool former = VFIRST || w == 0;
    float dtb[4] = {0.f, 0.f, 0.f, 0.f};
    if (p.use_gate && p.dt_bias && former) {
#pragma unroll
        for (int c = 0; c < (VFIRST ? 4 : 2); ++c) dtb[c] = p.dt_bias[hv * DK + col + c];
    }
    float gp[4] = {0.f, 0.f, 0.f, 0.f};  // G_{t-1} of the cumsum form
    const bool vlane = VFIRST ? t < 32 : true;  // V-first: threads that stage v

    TokRaw cur, nxt;
    const int len = ONE ? 1 : sp.len;
    if (len > 0) load_tok<VFIRST>(p, sp, 0, h, hv, t, cur);
    for (int tt = 0; tt < len; ++tt) {
        if (!ONE && tt + 1 < len) load_tok<VFIRST>(p, sp, tt + 1, h, hv, t, nxt);
        const int64_t rv = (sp.tok0 + tt) * HV + hv;
        const bool chunk_start = (tt % BT) == 0;
        float beta = cur.beta;
        if (p.use_beta_sigmoid) beta = sigmoid_precise(beta);

        if constexpr (VFIRST) {
            // this thread's columns of q^, k^ and the decay
            float qv[4] = {lo16(cur.q.x), hi16(cur.q.x), lo16(cur.q.y), hi16(cur.q.y)};
            float kv[4] = {lo16(cur.k.x), hi16(cur.k.x), lo16(cur.k.y), hi16(cur.k.y)};
            if (p.use_l2norm) {
                float sq = 0.f, sk = 0.f;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    sq = fmaf(qv[c], qv[c], sq);
                    sk = fmaf(kv[c], kv[c], sk);
                }
                const float nq = sqrtf(half_sum(sq) + L2_EPS);
                const float nk = sqrtf(half_sum(sk) + L2_EPS);
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    qv[c] /= nq;
                    kv[c] /= nk;
                }
            }
            float a[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) a[c] = decay_of(p, cur.g[c], ea, dtb[c], gp[c], chunk_start);
            float* sv = s_v[tt & 1];
            if (vlane)
                *reinterpret_cast<f32x4*>(sv + 4 * t) =
                    f32x4{lo16(cur.v.x), hi16(cur.v.x), lo16(cur.v.y), hi16(cur.v.y)};
            __syncthreads();
            float ov = 0.f;  // o of row 8 * j + hw, kept by lane j < 16
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float part = 0.f;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    S[i][c] *= a[c];
                    part = fmaf(S[i][c], kv[c], part);
                }
                const float pred = half_sum(part);
                const float vnew = beta * (sv[8 * i + hw] - pred);
                float po = 0.f;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    S[i][c] = fmaf(vnew, kv[c], S[i][c]);
                    po = fmaf(S[i][c], qv[c], po);
                }
                const float o = half_sum(po);
                if (j == i) ov = o;
            }
            if (j < 16) store_o(p, rv * DK + 8 * j + hw, p.scale * ov);
        } else {
            // wave 0 forms the token's decay, k^ and q^ for the work-group
            if (w == 0) {
                float q0 = lo16(cur.q.x), q1 = hi16(cur.q.x);
                float k0 = lo16(cur.k.x), k1 = hi16(cur.k.x);
                if (p.use_l2norm) {
                    float sq = fmaf(q0, q0, q1 * q1), sk = fmaf(k0, k0, k1 * k1);
                    sq = half_sum(sq);
                    sk = half_sum(sk);
                    sq += __shfl_xor(sq, 32, 64);
                    sk += __shfl_xor(sk, 32, 64);
                    const float nq = sqrtf(sq + L2_EPS), nk = sqrtf(sk + L2_EPS);
                    q0 /= nq; q1 /= nq;
                    k0 /= nk; k1 /= nk;
                }
                const int e = 2 * t;
                s_vec[0][e] = decay_of(p, cur.g[0], ea, dtb[0], gp[0], chunk_start);
                s_vec[0][e + 1] = decay_of(p, cur.g[1], ea, dtb[1], gp[1], chunk_start);
                s_vec[1][e] = k0;
                s_vec[1][e + 1] = k1;
                s_vec[2][e] = q0;
                s_vec[2][e + 1] = q1;
            }
            __syncthreads();
            float kv[16], qv[16];
            float part[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int k = 8 * i + hw;
                const float a = s_vec[0][k];
                kv[i] = s_vec[1][k];
                qv[i] = s_vec[2][k];
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    S[i][c] *= a;
                    part[c] = fmaf(S[i][c], kv[i], part[c]);
                }
            }
            // S k^ over this thread's 16 k, then the two half-waves of the
            // wave, then the four waves
#pragma unroll
            for (int c = 0; c < 4; ++c) part[c] += __shfl_xor(part[c], 32, 64);
            if ((t & 32) == 0)
                *reinterpret_cast<f32x4*>(&s_red[0][w][4 * j]) = f32x4{part[0], part[1], part[2], part[3]};
            __syncthreads();
            const float vv[4] = {lo16(cur.v.x), hi16(cur.v.x), lo16(cur.v.y), hi16(cur.v.y)};
            float vnew[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int v = 4 * j + c;
                const float pred = s_red[0][0][v] + s_red[0][1][v] + s_red[0][2][v] + s_red[0][3][v];
                vnew[c] = beta * (vv[c] - pred);
            }
            float po[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 16; ++i) {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    S[i][c] = fmaf(vnew[c], kv[i], S[i][c]);
                    po[c] = fmaf(S[i][c], qv[i], po[c]);
                }
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) po[c] += __shfl_xor(po[c], 32, 64);
            if ((t & 32) == 0)
                *reinterpret_cast<f32x4*>(&s_red[1][w][4 * j]) = f32x4{po[0], po[1], po[2], po[3]};
            __syncthreads();
            if (t < 32) {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int v = 4 * j + c;
                    const float o = s_red[1][0][v] + s_red[1][1][v] + s_red[1][2][v] + s_red[1][3][v];
                    store_o(p, rv * DK + v, p.scale * o);
                }
            }
        }
        if (!ONE && tt + 1 < len) cur = nxt;
    }

    if (p.ht) {
        float* ht = p.ht + sbase;
#pragma unroll
        for (int i = 0; i < 16; ++i) *reinterpret_cast<f32x4*>(ht + 1024 * i + 4 * t) = S[i];
    }
}

}  // namespace

hipError_t launch_recurrent(const Params& p, hipStream_t stream) {
    const int64_t grid = (int64_t)(p.cu_seqlens ? p.N : p.B) * p.HV;
    const bool one = !p.cu_seqlens && p.T == 1;
    auto kern = p.h0_v_first ? (one ? recurrent_kernel<true, true> : recurrent_kernel<true, false>)
                             : (one ? recurrent_kernel<false, true> : recurrent_kernel<false, false>);
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(RT), 0, stream, p);
    return hipGetLastError();
}

}  // namespace kda
