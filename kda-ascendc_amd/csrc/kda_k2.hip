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

// Records are streamed through an LDS ring of RING slots with the gfx950
// direct global->LDS loads (global_load_lds_dwordx4: 64 lanes x 16 B =
// 1 KiB per instruction, 17 per record), issued RING-1 chunks ahead of use.
// The loads complete in issue order, so before reading slot c the wave
// waits until at most 17 * (chunks issued after c) loads are outstanding;
// stores counted in the same counter only lengthen that wait.
constexpr int RING = 4;
constexpr int LOADS_PER_REC = REC_BYTES / 1024;
static_assert(LOADS_PER_REC * 1024 == REC_BYTES, "record must be whole KiB");

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ void wait_chunks_in_flight(int n_after) {
    static_assert(RING == 4, "wait ladder covers RING - 1 = 3 chunks");
    if (n_after >= 3) {
        wait_vmcnt<3 * LOADS_PER_REC>();
    } else if (n_after == 2) {
        wait_vmcnt<2 * LOADS_PER_REC>();
    } else if (n_after == 1) {
        wait_vmcnt<LOADS_PER_REC>();
    } else {
        wait_vmcnt<0>();
    }
}

__device__ __forceinline__ void issue_chunk(const uint8_t* __restrict__ src, uint8_t* slot, int lane) {
#pragma unroll
    for (int i = 0; i < LOADS_PER_REC; ++i)
        __builtin_amdgcn_global_load_lds(src + i * 1024 + lane * 16, slot + i * 1024, 16, 0, 0);
}

__global__ __launch_bounds__(64) void k2_kernel(Params p) {
    __shared__ __attribute__((aligned(1024))) uint8_t ring[RING * REC_BYTES];

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
    for (int d = 0; d < RING - 1; ++d)
        if (d < NT) issue_chunk(rec + (int64_t)d * REC_BYTES, ring + d * REC_BYTES, lane);

    for (int c = 0; c < NT; ++c) {
        const int cn = c + RING - 1;
        if (cn < NT) issue_chunk(rec + (int64_t)cn * REC_BYTES, ring + (cn % RING) * REC_BYTES, lane);
        wait_chunks_in_flight(min(RING - 1, NT - 1 - c));
        const uint8_t* slot = ring + (c % RING) * REC_BYTES;

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
            const u32x4 wj = *reinterpret_cast<const u32x4*>(slot + REC_W + j * 1024 + lane * 16);
            const u32x4 qj = *reinterpret_cast<const u32x4*>(slot + REC_QG + j * 1024 + lane * 16);
            vacc = mfma_bf16_16x16x32(as_bf16x8(wj), hc[j], vacc);
            oacc = mfma_bf16_16x16x32(as_bf16x8(qj), hc[j], oacc);
        }
        // v_new[4*q4 + i][v] = u - w @ hc^T, rounded to bf16 (kernels.py:261-266).
        const u32x2 uu = *reinterpret_cast<const u32x2*>(slot + REC_U + vt * 512 + lane * 8);
        const float u0 = __builtin_bit_cast(float, uu.x << 16);
        const float u1 = __builtin_bit_cast(float, uu.x & 0xffff0000u);
        const float u2 = __builtin_bit_cast(float, uu.y << 16);
        const float u3 = __builtin_bit_cast(float, uu.y & 0xffff0000u);
        const u32x2 vnb = {pack2(u0 - vacc[0], u1 - vacc[1]), pack2(u2 - vacc[2], u3 - vacc[3])};
        const i16x4 vn = as_i16x4(vnb);

        // o = scale * qg @ hc^T + Aqk @ v_new (kernels.py:268-279).
        const u32x2 aq = *reinterpret_cast<const u32x2*>(slot + REC_AQK + lane * 8);
        oacc = oacc * p.scale;
        oacc = mfma_bf16_16x16x16(as_i16x4(aq), vn, oacc);

        // S = S * 2^G_last + (kg^T @ v_new)^T (kernels.py:281-294).
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const u32x4 kg = *reinterpret_cast<const u32x4*>(slot + REC_KG + j * 1024 + lane * 16);
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
                const int kt = 2 * j + h2;
                const f32x4 dc = *reinterpret_cast<const f32x4*>(slot + REC_DECAY + kt * 64 + q4 * 16);
                const u32x2 kgt = h2 ? u32x2{kg.z, kg.w} : u32x2{kg.x, kg.y};
                St[kt] = mfma_bf16_16x16x16(as_i16x4(kgt), vn, St[kt] * dc);
            }
        }

        const int tbase = c * BT + 4 * q4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (tbase + i < T) p.o[(((int64_t)b * T + tbase + i) * H + h) * DK + v] = f2bf(oacc[i]);
        }
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
