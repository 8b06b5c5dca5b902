// Stage-2 helpers shared by the stage-2 kernels (kda_k2.hip: one value
// tile per work-group; kda_k2w.hip: several): the record ring's direct
// buffer->LDS loads and waits, the chunk barrier, the decay broadcast and the
// fp32 state slices of a value tile.
#pragma once

#include "kda_common.h"

namespace kda {
namespace {

typedef __attribute__((address_space(3))) uint8_t lds_u8;

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N));
}

// Buffer descriptor word 3 for raw byte-addressed buffers on gfx9-family
// parts (gfx950 included).
constexpr int BUF_DWORD3 = 0x00020000;

// Lane (x, q4) reads 2^G_last at [kt = x/2][q4][i = 2*(x%2) .. +1].
__device__ __forceinline__ uint32_t decay_offset(int lane) {
    const int x = lane & 15, q4 = lane >> 4;
    return REC_DECAY + (x >> 1) * 64 + q4 * 16 + (x & 1) * 8;
}

// Scales the state tile kt by its decay: element i of lane (x, q4) takes
// 2^G_last[16*kt + 4*q4 + i] from lane 2*kt + i/2 of its row (DPP
// row_newbcast, row_bcast in kda_common.h), component i % 2.
template <int KT>
__device__ __forceinline__ f32x4 decay_tile(f32x4 st, f32x2 dc) {
    return f32x4{st[0] * row_bcast<2 * KT>(dc.x), st[1] * row_bcast<2 * KT>(dc.y),
                 st[2] * row_bcast<2 * KT + 1>(dc.x), st[3] * row_bcast<2 * KT + 1>(dc.y)};
}

// s_waitcnt immediates on gfx9-family parts: vmcnt field (bits 3:0 and
// 15:14) and expcnt (bits 6:4) at their maxima, lgkmcnt (bits 11:8) 0 or 15.
constexpr int WAITCNT_LGKM0 = 0xC07F;
constexpr int WAITCNT_LGKM15 = 0xCF7F;

// Chunk barrier: the wave's LDS accesses are complete, then all waves of
// the work-group meet.  The wait and barrier are one inline asm block whose memory clobber
// keeps every LDS access on its side; as asm, the barrier carries no
// implied wait on the output wave's stores.  The builtin wait after it
// costs nothing (the count is already zero) but tells the compiler so,
// which keeps it from adding conservative waits for LDS reads issued
// before the barrier.
__device__ __forceinline__ void chunk_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_s_waitcnt(WAITCNT_LGKM0);
}

// The copy wave's side of the barrier: no clobber, so the compiler adds no
// wait for its loads in flight.
__device__ __forceinline__ void copy_barrier() { asm volatile("s_barrier"); }

// Fp32 state slice of this lane from `src` ([V, K] if v_first, else
// [K, V]; null: zeros): St[kt][i] = S[v][16*kt + 4*q4 + i].
__device__ __forceinline__ void load_state_from(const float* src, bool v_first, int v, int q4,
                                                f32x4 (&St)[8]) {
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
        St[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (src) {
            const int k0 = 16 * kt + 4 * q4;
            if (v_first) {
                St[kt] = *reinterpret_cast<const f32x4*>(src + (int64_t)v * DK + k0);
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) St[kt][i] = src[(int64_t)(k0 + i) * DK + v];
            }
        }
    }
}

__device__ __forceinline__ void store_state_to(float* dst, bool v_first, int v, int q4,
                                               const f32x4 (&St)[8]) {
    if (!dst) return;
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
        const int k0 = 16 * kt + 4 * q4;
        if (v_first) {
            *reinterpret_cast<f32x4*>(dst + (int64_t)v * DK + k0) = St[kt];
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) dst[(int64_t)(k0 + i) * DK + v] = St[kt][i];
        }
    }
}

// S^T tiles of this lane: St[kt][i] = S[v][16*kt + 4*q4 + i], v = 16*vt + lane%16.
// (The layout and presence tests are outside the loads, so that all of them
// are in flight before the first wait.)
__device__ __forceinline__ void load_state(const Params& p, int64_t sbase, int v, int q4,
                                           f32x4 (&St)[8]) {
    if (!p.h0) {
#pragma unroll
        for (int kt = 0; kt < 8; ++kt) St[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
    } else if (p.h0_v_first) {
#pragma unroll
        for (int kt = 0; kt < 8; ++kt)
            St[kt] = *reinterpret_cast<const f32x4*>(p.h0 + sbase + (int64_t)v * DK + 16 * kt + 4 * q4);
    } else {
#pragma unroll
        for (int kt = 0; kt < 8; ++kt) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                St[kt][i] = p.h0[sbase + (int64_t)(16 * kt + 4 * q4 + i) * DK + v];
        }
    }
}

__device__ __forceinline__ void store_state(const Params& p, int64_t sbase, int v, int q4,
                                            const f32x4 (&St)[8]) {
    if (!p.ht) return;
    if (p.ht_v_first) {
#pragma unroll
        for (int kt = 0; kt < 8; ++kt)
            *reinterpret_cast<f32x4*>(p.ht + sbase + (int64_t)v * DK + 16 * kt + 4 * q4) = St[kt];
    } else {
#pragma unroll
        for (int kt = 0; kt < 8; ++kt) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                p.ht[sbase + (int64_t)(16 * kt + 4 * q4 + i) * DK + v] = St[kt][i];
        }
    }
}

}  // namespace
}  // namespace kda
