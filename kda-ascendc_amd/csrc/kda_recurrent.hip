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
// One work-group of two waves per (batch, value head).  Lane v of the
// work-group owns row v of S in 128 VGPRs, so the per-token products
// S k^ and S q^ are per-lane dot products with no cross-lane reduction.
// Each token's decay, k^ and q^ (128 values each) are formed by every wave
// for itself (lane l: elements 2l, 2l+1; the l2 norms by a wave-wide
// butterfly sum) into its own LDS area and read back as broadcasts.
// A V-first state ([V, K], row v contiguous) is moved between HBM and the
// lanes' rows through LDS: the work-group reads and writes it with
// coalesced 16-byte accesses (each wave instruction covers 1 KiB of
// consecutive memory), and each lane reads or writes its row in LDS, rows
// padded to 132 floats so that the 16-byte row accesses of 16 consecutive
// lanes fall in distinct banks.  Read directly, lane v's 16-byte pieces of
// row v sit 512 bytes apart across the wave and every load instruction
// touches 64 cache lines.  A K-first state ([K, V]) is already coalesced
// for this lane-per-row layout (lane v reads S[k][v] for each k).
// Grouped value heads (GVA): value head hv reads q/k head hv / (HV / H)
// (kernels.py:88).  Varlen: one work-group per (sequence, value head), over
// the sequence's tokens, with states [N, HV, ...].
#include "kda_common.h"

namespace kda {

namespace {

__device__ __forceinline__ float load_scalar(const void* base, int is_bf16, int64_t i) {
    return is_bf16 ? bf2f(static_cast<const uint16_t*>(base)[i])
                   : static_cast<const float*>(base)[i];
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m, 64);
    return x;
}

__device__ __forceinline__ float sigmoid_precise(float x) { return 1.0f / (1.0f + expf(-x)); }

constexpr int SROW = DK + 4;  // padded LDS row of the state, in floats
constexpr int NTHREADS = 128;

__global__ __launch_bounds__(NTHREADS) void recurrent_kernel(Params p) {
    const int HV = p.HV, H = p.H;
    const int bhv = blockIdx.x;  // (batch row or sequence) * HV + hv
    const int hv = bhv - (bhv / HV) * HV;
    const int h = hv / (HV / H);
    const SeqSpan sp = seq_span(p, bhv);
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int vrow = 64 * w + lane;  // this lane's row of S
    const int k0 = 2 * lane;         // this lane's two elements of the token vectors

    // Per wave: [0] decay, [1] k^, [2] q^ of the current token.
    __shared__ __attribute__((aligned(16))) float vec[2][3][DK];
    // A V-first state on its way in or out.
    __shared__ __attribute__((aligned(16))) float stage[DK * SROW];

    float S[DK];
    const int64_t sbase = (int64_t)bhv * DK * DK;
#pragma unroll
    for (int k = 0; k < DK; ++k) S[k] = 0.0f;
    if (p.h0) {
        if (p.h0_v_first) {
            // pass i: thread x moves floats 4 * (128 i + x) .. + 3
#pragma unroll 8
            for (int i = 0; i < DK * DK / (4 * NTHREADS); ++i) {
                const int e = 4 * (i * NTHREADS + (int)threadIdx.x);
                const f32x4 r = *reinterpret_cast<const f32x4*>(p.h0 + sbase + e);
                *reinterpret_cast<f32x4*>(stage + (e >> 7) * SROW + (e & (DK - 1))) = r;
            }
            __syncthreads();
#pragma unroll
            for (int k = 0; k < DK; k += 4) {
                const f32x4 r = *reinterpret_cast<const f32x4*>(stage + vrow * SROW + k);
                S[k] = r[0]; S[k + 1] = r[1]; S[k + 2] = r[2]; S[k + 3] = r[3];
            }
        } else {
#pragma unroll
            for (int k = 0; k < DK; ++k) S[k] = p.h0[sbase + (int64_t)k * DK + vrow];
        }
    }

    const float ea = p.use_gate ? expf(p.A_log[hv]) : 0.0f;
    float dtb0 = 0.0f, dtb1 = 0.0f;
    if (p.use_gate && p.dt_bias) {
        dtb0 = p.dt_bias[hv * DK + k0];
        dtb1 = p.dt_bias[hv * DK + k0 + 1];
    }

    float gp0 = 0.0f, gp1 = 0.0f;  // G_{t-1} of the cumsum form
    for (int t = 0; t < sp.len; ++t) {
        const int64_t rq = (sp.tok0 + t) * H + h;   // q/k row
        const int64_t rv = (sp.tok0 + t) * HV + hv; // v/g/beta/o row

        float q0 = bf2f(p.q[rq * DK + k0]), q1 = bf2f(p.q[rq * DK + k0 + 1]);
        float c0 = bf2f(p.k[rq * DK + k0]), c1 = bf2f(p.k[rq * DK + k0 + 1]);
        if (p.use_l2norm) {
            const float nq = sqrtf(wave_sum(q0 * q0 + q1 * q1) + L2_EPS);
            const float nk = sqrtf(wave_sum(c0 * c0 + c1 * c1) + L2_EPS);
            q0 /= nq; q1 /= nq;
            c0 /= nk; c1 /= nk;
        }
        const float g0 = load_scalar(p.g, p.g_bf16, rv * DK + k0);
        const float g1 = load_scalar(p.g, p.g_bf16, rv * DK + k0 + 1);
        float a0, a1;
        if (p.use_gate) {
            a0 = expf(p.lower_bound * sigmoid_precise(ea * (g0 + dtb0)));
            a1 = expf(p.lower_bound * sigmoid_precise(ea * (g1 + dtb1)));
        } else if (p.g_log) {
            a0 = expf(g0);
            a1 = expf(g1);
        } else {
            if (t % BT == 0) gp0 = gp1 = 0.0f;
            a0 = exp2f(g0 - gp0);
            a1 = exp2f(g1 - gp1);
            gp0 = g0;
            gp1 = g1;
        }
        vec[w][0][k0] = a0; vec[w][0][k0 + 1] = a1;
        vec[w][1][k0] = c0; vec[w][1][k0 + 1] = c1;
        vec[w][2][k0] = q0; vec[w][2][k0 + 1] = q1;

        float bt = load_scalar(p.beta, p.beta_bf16, rv);
        if (p.use_beta_sigmoid) bt = sigmoid_precise(bt);
        const float vt = bf2f(p.v[rv * DK + vrow]);

        // Lanes read what other lanes of the wave wrote: the wave barrier
        // keeps the compiler from moving reads above the writes, and one
        // wave's LDS operations execute in order.
        __builtin_amdgcn_wave_barrier();
        float pred = 0.0f;
#pragma unroll
        for (int k = 0; k < DK; ++k) {
            S[k] *= vec[w][0][k];
            pred = fmaf(S[k], vec[w][1][k], pred);
        }
        const float vnew = bt * (vt - pred);
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < DK; ++k) {
            S[k] = fmaf(vnew, vec[w][1][k], S[k]);
            acc = fmaf(S[k], vec[w][2][k], acc);
        }
        const float ot = p.scale * acc;
        if (p.o_fp32) {
            reinterpret_cast<float*>(p.o)[rv * DK + vrow] = ot;
        } else {
            p.o[rv * DK + vrow] = f2bf(ot);
        }
        // The next token's writes stay below this token's reads.
        __builtin_amdgcn_wave_barrier();
    }

    if (p.ht) {
        if (p.ht_v_first) {
            // Other lanes may still be reading their rows of a staged h0.
            __syncthreads();
#pragma unroll
            for (int k = 0; k < DK; k += 4)
                *reinterpret_cast<f32x4*>(stage + vrow * SROW + k) =
                    f32x4{S[k], S[k + 1], S[k + 2], S[k + 3]};
            __syncthreads();
#pragma unroll 8
            for (int i = 0; i < DK * DK / (4 * NTHREADS); ++i) {
                const int e = 4 * (i * NTHREADS + (int)threadIdx.x);
                *reinterpret_cast<f32x4*>(p.ht + sbase + e) =
                    *reinterpret_cast<const f32x4*>(stage + (e >> 7) * SROW + (e & (DK - 1)));
            }
        } else {
#pragma unroll
            for (int k = 0; k < DK; ++k) p.ht[sbase + (int64_t)k * DK + vrow] = S[k];
        }
    }
}

}  // namespace

hipError_t launch_recurrent(const Params& p, hipStream_t stream) {
    const int64_t grid = (int64_t)(p.cu_seqlens ? p.N : p.B) * p.HV;
    hipLaunchKernelGGL(recurrent_kernel, dim3((unsigned)grid), dim3(NTHREADS), 0, stream, p);
    return hipGetLastError();
}

}  // namespace kda
