// Stage 2 of the KDA BT=16 forward: the serial delta-rule recurrence.
//
// Follows kda_bt16_kernel_k2 (/root/reference/src/kda_bt16/kernels.py:187-302):
// per chunk,
//   hc    = bf16(S)
//   v_new = bf16(u - w @ hc^T)
//   o     = bf16(scale * (qg @ hc^T) + Aqk @ v_new)
//   S     = S * 2^G_last[None, :] + (kg^T @ v_new)^T
// with S the [V, K] fp32 state.  One 64-lane wave owns 16 value columns of
// one (batch, head) and keeps its slice of S transposed, S^T[k][v], as eight
// 16x16 fp32 accumulator tiles.  The 16x16 accumulator layout (lane
// v + 16*(k/4), item k%4) is exactly the B-operand layout of the 16x16x16
// bf16 matrix op, so bf16(S) feeds the next chunk's products straight from
// registers: the serial chain has no LDS traffic and no barrier.  Pairs of
// k-tiles form the 8-deep operands of the 16x16x32 op for w @ hc^T and
// qg @ hc^T; stage 1 stored w and qg in the matching k order.
#include "kda_common.h"

namespace kda {

namespace {

struct Chunk {
    u32x4 w[4];
    u32x4 qg[4];
    u32x2 kg[8];
    u32x2 u;
    u32x2 aqk;
    f32x4 decay[8];
};

__device__ __forceinline__ void load_chunk(const uint8_t* __restrict__ rec, int lane, int q4, int vt,
                                           Chunk& ch) {
    const u32x4* w = reinterpret_cast<const u32x4*>(rec + REC_W + lane * 64);
    const u32x4* qg = reinterpret_cast<const u32x4*>(rec + REC_QG + lane * 64);
    const u32x2* kg = reinterpret_cast<const u32x2*>(rec + REC_KG + lane * 64);
    const f32x4* dc = reinterpret_cast<const f32x4*>(rec + REC_DECAY + q4 * 128);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        ch.w[j] = w[j];
        ch.qg[j] = qg[j];
    }
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
        ch.kg[kt] = kg[kt];
        ch.decay[kt] = dc[kt];
    }
    ch.u = *reinterpret_cast<const u32x2*>(rec + REC_U + vt * 512 + lane * 8);
    ch.aqk = *reinterpret_cast<const u32x2*>(rec + REC_AQK + lane * 8);
}

__global__ __launch_bounds__(64) void k2_kernel(Params p) {
    const int lane = threadIdx.x;
    const int x = lane & 15;  // value column inside the tile
    const int q4 = lane >> 4;
    const int H = p.H, T = p.T, NT = p.NT;
    const int nbh = p.B * H;

    // Work-group -> (head, value tile), XCD aware: consecutive work-group ids
    // go to different XCDs round-robin, so the 8 tiles of one head get ids
    // of one residue class mod 8 and share that XCD's L2 for the records.
    const int wg = blockIdx.x;
    const int lin = (wg & 7) * nbh + (wg >> 3);
    const int bh = lin >> 3;
    const int vt = lin & 7;
    const int b = bh / H, h = bh - (bh / H) * H;
    const int v = 16 * vt + x;

    // S^T tiles: St[kt][i] = S[v][16*kt + 4*q4 + i].
    f32x4 St[8];
    const int64_t sbase = (int64_t)bh * DK * DK;
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
        St[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (p.h0) {
            const int k0 = 16 * kt + 4 * q4;
            if (p.state_v_first) {
                St[kt] = *reinterpret_cast<const f32x4*>(p.h0 + sbase + (int64_t)v * DK + k0);
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) St[kt][i] = p.h0[sbase + (int64_t)(k0 + i) * DK + v];
            }
        }
    }

    const uint8_t* rec = p.ws + (int64_t)bh * NT * REC_BYTES;
    Chunk cur;
    load_chunk(rec, lane, q4, vt, cur);

    for (int c = 0; c < NT; ++c) {
        Chunk nxt;
        if (c + 1 < NT) load_chunk(rec + (int64_t)(c + 1) * REC_BYTES, lane, q4, vt, nxt);

        // hc = bf16(S), as 16x16x32 B operands (k-tiles 2j and 2j+1).
        bf16x8 hc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const u32x4 pk = {pack2(St[2 * j][0], St[2 * j][1]), pack2(St[2 * j][2], St[2 * j][3]),
                              pack2(St[2 * j + 1][0], St[2 * j + 1][1]),
                              pack2(St[2 * j + 1][2], St[2 * j + 1][3])};
            hc[j] = as_bf16x8(pk);
        }
        f32x4 vacc = {0.f, 0.f, 0.f, 0.f};
        f32x4 oacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            vacc = mfma_bf16_16x16x32(as_bf16x8(cur.w[j]), hc[j], vacc);
            oacc = mfma_bf16_16x16x32(as_bf16x8(cur.qg[j]), hc[j], oacc);
        }
        // v_new[4*q4 + i][v] = u - w @ hc^T, rounded to bf16 (kernels.py:261-266).
        const float u0 = __builtin_bit_cast(float, cur.u.x << 16);
        const float u1 = __builtin_bit_cast(float, cur.u.x & 0xffff0000u);
        const float u2 = __builtin_bit_cast(float, cur.u.y << 16);
        const float u3 = __builtin_bit_cast(float, cur.u.y & 0xffff0000u);
        const u32x2 vnb = {pack2(u0 - vacc[0], u1 - vacc[1]), pack2(u2 - vacc[2], u3 - vacc[3])};
        const i16x4 vn = as_i16x4(vnb);

        // o = scale * qg @ hc^T + Aqk @ v_new (kernels.py:268-279).
        oacc = oacc * p.scale;
        oacc = mfma_bf16_16x16x16(as_i16x4(cur.aqk), vn, oacc);

        // S = S * 2^G_last + (kg^T @ v_new)^T (kernels.py:281-294).
#pragma unroll
        for (int kt = 0; kt < 8; ++kt) {
            St[kt] = St[kt] * cur.decay[kt];
            St[kt] = mfma_bf16_16x16x16(as_i16x4(cur.kg[kt]), vn, St[kt]);
        }

        const int tbase = c * BT + 4 * q4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (tbase + i < T) p.o[(((int64_t)b * T + tbase + i) * H + h) * DK + v] = f2bf(oacc[i]);
        }
        if (c + 1 < NT) cur = nxt;
    }

    if (p.ht) {
#pragma unroll
        for (int kt = 0; kt < 8; ++kt) {
            const int k0 = 16 * kt + 4 * q4;
            if (p.state_v_first) {
                *reinterpret_cast<f32x4*>(p.ht + sbase + (int64_t)v * DK + k0) = St[kt];
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) p.ht[sbase + (int64_t)(k0 + i) * DK + v] = St[kt][i];
            }
        }
    }
}

}  // namespace

hipError_t launch_k2(const Params& p, hipStream_t stream) {
    const int64_t grid = (int64_t)p.B * p.H * 8;
    hipLaunchKernelGGL(k2_kernel, dim3((unsigned)grid), dim3(64), 0, stream, p);
    return hipGetLastError();
}

}  // namespace kda
