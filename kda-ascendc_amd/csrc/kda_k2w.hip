// Stage 2 of the KDA BT=16 forward for throughput-bound shapes: several
// value tiles per work-group sharing one record stream.
//
// Same recurrence as kda_k2.hip (kernels.py:225-302), per chunk
//   hc    = bf16(S)
//   v_new = bf16(u - w @ hc^T)
//   o     = bf16(scale * (qg @ hc^T) + Aqk @ v_new)
//   S     = S * 2^G_last[None, :] + (kg^T @ v_new)^T
// with identical arithmetic, so o and ht are bit for bit those of
// kda_k2.hip.  What changes is who does the work:
//
// kda_k2.hip gives each (sequence, head, 16 value columns) a work-group of
// its own, which pulls the 13 KiB of the record that every value tile needs
// through its CU's texture path: with more such work-groups than CUs, that
// repeated pull (8x per head and chunk) is what paces the kernel.  Here a
// work-group takes TPW value tiles of one (sequence, head):
//   * one copy wave streams each chunk's record once -- the shared 13 KiB
//     and the TPW u slices -- into an LDS ring (direct buffer->LDS loads);
//   * TPW / TW compute waves each own TW (1 or 2) value tiles.  A compute
//     wave keeps its tiles' state slices in registers (S^T as eight 16x16
//     fp32 accumulator tiles each, the layout of kda_k2.hip) and forms their
//     v_new, o and state updates itself: no hand-off through LDS.  The
//     operands every tile shares (w, qg, kg, Aqk, the decay) are read from
//     LDS once per wave, at the start of the chunk (behind the packing of
//     hc, which needs only the state): with two tiles a wave reads them once
//     for both, with one tile twice the waves issue the work.
// The waves meet at one barrier per chunk.
#include "kda_common.h"
#include "kda_k2_shared.h"
#include "kda_k2w_step.h"

namespace kda {

namespace {

constexpr int SHARED_LOADS_W = REC_SHARED / 1024;  // 13

// Ring geometry of a TPW-tile work-group.  A slot holds the shared 13 KiB
// and the TPW u slices of this work-group's tiles (contiguous in the
// record).  The copy wave issues chunk c + LEAD during chunk c and, before
// the barrier that ends chunk c, waits for chunk c + 1, which the compute
// waves read during chunk c + 1.  Chunk j's slot is read during chunk j and
// refilled with chunk j + RING during chunk j + RING - LEAD = j + 1, after
// that read.  Direct loads count in the 6-bit vmcnt: LEAD chunks of loads
// must fit in 63.
template <int TPW, int TW>
struct WideGeom {
    static_assert(TPW == 2 || TPW == 4 || TPW == 8, "two, four or eight value tiles");
    static_assert(TW == 1 || TW == 2, "one or two value tiles per compute wave");
    static constexpr int NCW = TPW / TW;                   // compute waves
    static constexpr int NL = SHARED_LOADS_W + TPW / 2;    // 1 KiB loads per chunk
    static constexpr int LEAD = 4 * NL <= 63 ? 4 : 3;
    static constexpr int RING = LEAD + 1;
    static constexpr int SLOT = REC_SHARED + TPW * 512;
    static constexpr int THREADS = 64 * (NCW + 1);
    static_assert(LEAD * NL <= 63, "vmcnt is a 6-bit count");
};

// Chunks c .. c + N - 1 (those below NT), with the ring slot of chunk c as
// the compile-time S (every LDS offset a constant).
template <int TPW, int TW, int S, int N>
__device__ __forceinline__ void wide_round(const WideCtx& cx, int c, f32x4 (&SA)[8], f32x4 (&SB)[8],
                                           const uint8_t* ring, int ut) {
    using G = WideGeom<TPW, TW>;
    if (c >= cx.NT) return;
    if constexpr (TW == 2) {
        BarrierHooks hk;
        wide_step(cx, c, SA, SB, ring + S * G::SLOT, ut, hk);
    } else {
        wide1_step(cx, c, SA, ring + S * G::SLOT, ut);
    }
    if constexpr (N > 1) wide_round<TPW, TW, (S + 1) % G::RING, N - 1>(cx, c + 1, SA, SB, ring, ut);
}

// Copy wave: the NL loads of one chunk, the shared part then this
// work-group's u slices.
template <int NL>
__device__ __forceinline__ void issue_wide_chunk(__amdgpu_buffer_rsrc_t rs, uint32_t chunk_off,
                                                 lds_u8* slot, uint32_t u_off, uint32_t voff16) {
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        const uint32_t src = i < SHARED_LOADS_W ? chunk_off + i * 1024
                                                : chunk_off + u_off + (i - SHARED_LOADS_W) * 1024;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_u8*)(slot + i * 1024), 16, voff16, src,
                                                 0, 0);
    }
}

// Wait until the chunk followed by `n_after` issued chunks has landed.
template <int N, int NL>
__device__ __forceinline__ void wide_wait_ladder(int n_after) {
    if constexpr (N == 0) {
        wait_vmcnt<0>();
    } else {
        if (n_after >= N) {
            wait_vmcnt<N * NL>();
        } else {
            wide_wait_ladder<N - 1, NL>(n_after);
        }
    }
}

template <int TPW, int TW, int S>
__device__ __forceinline__ void wide_copy_round(__amdgpu_buffer_rsrc_t rs, lds_u8* ring, int c,
                                                int NT, uint32_t u_off, uint32_t voff16) {
    using G = WideGeom<TPW, TW>;
    if (c >= NT) return;
    if (c + G::LEAD < NT)
        issue_wide_chunk<G::NL>(rs, (uint32_t)(c + G::LEAD) * REC_BYTES,
                                ring + ((S + G::LEAD) % G::RING) * G::SLOT, u_off, voff16);
    // chunk c + 1 is read by the compute waves after this barrier
    if (c + 1 < NT) wide_wait_ladder<G::LEAD - 1, G::NL>(min(G::LEAD - 1, NT - 2 - c));
    copy_barrier();
    if constexpr (S + 1 < G::RING) wide_copy_round<TPW, TW, S + 1>(rs, ring, c + 1, NT, u_off, voff16);
}

// Work-group (sequence, value head, slice of TPW value tiles): grid padded
// to a multiple of 8 * (8 / TPW) and mapped XCD-aware, so that the slices
// of one (sequence, head) share an XCD and its L2 for the records.
template <int TPW, int TW>
__global__ __launch_bounds__((WideGeom<TPW, TW>::THREADS)) void k2w_kernel(Params p) {
    using G = WideGeom<TPW, TW>;
    __shared__ __attribute__((aligned(1024))) uint8_t ring[G::RING * G::SLOT];
    constexpr int NSL = 8 / TPW;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nbh = (p.cu_seqlens ? p.N : p.B) * p.HV;
    const int total = nbh * NSL;
    const int padded = (total + 8 * NSL - 1) / (8 * NSL) * (8 * NSL);
    const int wg = blockIdx.x;
    const int lin = (wg & 7) * (padded >> 3) + (wg >> 3);
    if (lin >= total) return;  // padding: the whole work-group leaves before any barrier
    const int bh = lin / NSL;
    const int slice = lin - bh * NSL;
    const int hv = bh - (bh / p.HV) * p.HV;
    const SeqSpan sp = seq_span(p, bh);
    const int64_t sbase = (int64_t)bh * DK * DK;

    if (wave < G::NCW) {
        const int ut = TW * wave;              // first of this wave's tiles in the slice
        const int vt = slice * TPW + ut;       // its value tile
        const int q4 = lane >> 4;
        const int va = 16 * vt + (lane & 15);  // this lane's state row (V index) of tile A
        f32x4 SA[8], SB[8];
        load_state(p, sbase, va, q4, SA);
        if (TW == 2) load_state(p, sbase, va + 16, q4, SB);
        if (sp.nt == 0) {  // an empty sequence: the final state is the initial state
            store_state(p, sbase, va, q4, SA);
            if (TW == 2) store_state(p, sbase, va + 16, q4, SB);
            __builtin_amdgcn_endpgm();
        }
        WideCtx cx;
        cx.scale = p.scale;
        cx.NT = sp.nt;
        cx.T = sp.len;
        cx.lane = lane;
        cx.q4 = q4;
        const int col = 4 * ((lane & 15) >> 2);
        cx.obase[0] = p.o + (sp.tok0 * p.HV + hv) * DK + 16 * vt + col;
        cx.obase[1] = cx.obase[0] + 16;
        cx.orow_stride = (int64_t)p.HV * DK;
        chunk_barrier();  // chunk 0 is in the ring
        for (int c = 0; c < cx.NT; c += G::RING) wide_round<TPW, TW, 0, G::RING>(cx, c, SA, SB, ring, ut);
        store_state(p, sbase, va, q4, SA);
        if (TW == 2) store_state(p, sbase, va + 16, q4, SB);
        __builtin_amdgcn_endpgm();
    }
    // copy wave
    if (sp.nt == 0) __builtin_amdgcn_endpgm();
    const int NT = sp.nt;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        p.ws + sp.rec0 * REC_BYTES, (short)0, NT * REC_BYTES, BUF_DWORD3);
    const uint32_t voff16 = lane * 16;
    const uint32_t u_off = REC_U + slice * TPW * 512;
    lds_u8* rl = (lds_u8*)ring;
#pragma unroll
    for (int d = 0; d < G::LEAD; ++d)
        if (d < NT) issue_wide_chunk<G::NL>(rs, (uint32_t)d * REC_BYTES, rl + d * G::SLOT, u_off, voff16);
    // chunk 0 before the first barrier
    wide_wait_ladder<G::LEAD - 1, G::NL>(min(G::LEAD, NT) - 1);
    copy_barrier();
    for (int c = 0; c < NT; c += G::RING) wide_copy_round<TPW, TW, 0>(rs, rl, c, NT, u_off, voff16);
    __builtin_amdgcn_endpgm();
}

}  // namespace

// Value tiles per work-group of the wide stage 2, or 0 for kda_k2.hip's one
// tile per work-group: the caller's p.k2_tiles when set, else the fewest
// tiles (1, 2, 4, 8) that keep the (sequences x heads x 8 / tiles)
// work-groups within one per CU.  A second round of work-groups costs more
// than wider ones: B=2 T=8192 H=32 (64 pairs) runs stage 2 in 196 us with 2
// tiles, 233 with 4 and 321 with 1; B=4 T=4096 H=32 (128 pairs) in 156 us
// with 4 tiles, 193 with 2 and 198 with 8.
int k2_wide_tiles(const Params& p, int ncu) {
    const int64_t nbh = (int64_t)(p.cu_seqlens ? p.N : p.B) * p.HV;
    if (p.k2_tiles != 0) return p.k2_tiles == 1 ? 0 : p.k2_tiles;
    if (nbh * 8 <= ncu) return 0;
    if (nbh * 4 <= ncu) return 2;
    if (nbh * 2 <= ncu) return 4;
    return 8;
}

namespace {
template <int TPW, int TW>
void launch_w(const Params& p, int64_t grid, hipStream_t stream) {
    hipLaunchKernelGGL((k2w_kernel<TPW, TW>), dim3((unsigned)grid), dim3(WideGeom<TPW, TW>::THREADS), 0,
                       stream, p);
}
}  // namespace

hipError_t launch_k2_wide(const Params& p, int tpw, hipStream_t stream) {
    const int64_t nbh = (int64_t)(p.cu_seqlens ? p.N : p.B) * p.HV;
    const int64_t nsl = 8 / tpw;
    const int64_t padded = (nbh * nsl + 8 * nsl - 1) / (8 * nsl) * (8 * nsl);
    // One tile per compute wave issues the work of 2 or 4 tiles from twice
    // the waves (B=1 T=8192 H=96, 4 tiles: stage 2 284 against 354 us);
    // with 8 tiles, 9 waves gained nothing over 5 (B=16 T=2048 H=32: 317 us
    // both), so two tiles per wave there.  p.k2_wave_tiles overrides.
    const int tw = p.k2_wave_tiles != 0 ? p.k2_wave_tiles : (tpw == 8 ? 2 : 1);
    switch (tpw * 4 + tw) {
        case 2 * 4 + 1: launch_w<2, 1>(p, padded, stream); break;
        case 4 * 4 + 1: launch_w<4, 1>(p, padded, stream); break;
        case 8 * 4 + 1: launch_w<8, 1>(p, padded, stream); break;
        case 2 * 4 + 2: launch_w<2, 2>(p, padded, stream); break;
        case 4 * 4 + 2: launch_w<4, 2>(p, padded, stream); break;
        default: launch_w<8, 2>(p, padded, stream); break;
    }
    return hipGetLastError();
}

}  // namespace kda
