// Stage 1 of the KDA BT=16 forward: everything that does not depend on the
// recurrent state, one 64-lane wave per (batch, head, 16-token chunk).
//
// Follows kda_bt16_kernel_k1 (/root/reference/src/kda_bt16/kernels.py:53-184)
// for the math and its bf16 rounding points, and additionally produces the
// per-chunk operands the reference recomputes inside its serial state loop
// (kernels.py:253-291): bf16(q^ * 2^G), bf16(k^ * 2^(G_last - G)) and
// 2^G_last.  Moving them here takes the l2norm and every exp2 off the
// serial chain of stage 2.
//
// Lane l owns row r = l & 15 of the chunk and the 32 columns
// {16*kt + 4*q4 + i} (q4 = l >> 4), so that
//   * row reductions (l2norm) are two cross-row shuffles,
//   * the column cumsum over the 16 rows is a DPP row scan,
//   * the fp32 grams run on 16x16x4 f32 matrix cores straight from
//     registers (any fixed assignment of columns to k-slots is a valid
//     reduction order), landing as Aqk[r][4*q4 + i] in lane (r, q4),
//   * w comes out of the matrix cores directly in stage 2's operand order.
#include "kda_k1_chunk.h"

namespace kda {

namespace {

// Three waves per SIMD (at most 168 VGPRs; the compiler spills two 8-byte
// values): each wave spends most of its life waiting on its loads, and a
// third wave per SIMD hides more of that than the two that 172 VGPRs allow.
//
// K1M (the record modes, below) other than K1_FWD also writes the backward
// record (kda_common.h) to p.ws_bwd: the same chunk quantities in the
// operand orders of the reverse state chain, from one read of the inputs,
// and the gram block to p.la.  Those modes run two waves per SIMD: they
// hold more.
// LDS of a work-group (one wave): k1_chunk's scratch.
__shared__ __attribute__((aligned(16))) float s_L[BT * BT];
__shared__ float s_X[BT * (BT + 1)];

// The (value head, chunk, sequence) of this work-group; false for a gap
// slot (wave-uniform, before any barrier).  With cu_seqlens, slot x of
// value head hv belongs to the sequence n with the largest
// floor(bos_n / 16) + n <= x; slots past its last chunk are gaps.  Fixed
// length: chunk-major, last chunk first, so the work-groups in flight
// together read whole token rows, and the records of the first chunks,
// which stage 2 starts with, are written last.
__device__ __forceinline__ bool block_chunk(const Params& p, int lane, int& hv, int& c, SeqSpan& sp) {
    const int HV = p.HV;
    if (p.cu_seqlens) {
        hv = blockIdx.x / p.NS;
        const int x = blockIdx.x - hv * p.NS;
        const int n = find_sequence(p, x, lane);
        sp = seq_span(p, n * HV + hv);
        c = (int)((int64_t)x - (sp.rec0 - (int64_t)hv * p.NS));
        return c >= 0 && c < sp.nt;
    }
    const int nbh = p.B * HV;
    const int bh = blockIdx.x % nbh;
    c = p.NT - 1 - (int)(blockIdx.x / nbh);
    hv = bh - (bh / HV) * HV;
    sp = seq_span(p, bh);
    return true;
}

// ALL_FULL: fixed-length batch with T a multiple of 16, so every chunk is
// full.  Otherwise every chunk takes the general path: both variants in one
// kernel would not fit the register budget of three waves per SIMD.
template <int K1M, bool ALL_FULL, bool GB16>
__global__ __launch_bounds__(64)
__attribute__((amdgpu_waves_per_eu(K1M != K1_FWD ? 2 : 3))) void k1_kernel(Params p) {
    int hv, c;
    SeqSpan sp;
    if (!block_chunk(p, threadIdx.x, hv, c, sp)) return;
    k1_chunk<K1M, ALL_FULL, GB16>(p, hv, c, sp, s_L, s_X, p.ws + (sp.rec0 + c) * REC_BYTES);
}

// The dO operand of each backward record that a training forward saved
// without it (K1_SAVE): [vt][lane][i] = dO[4*q4 + i][16*vt + r], rows past
// the sequence zero, as K1_BOTH writes it.
__global__ __launch_bounds__(64) void k1_dout_kernel(Params p) {
    const int lane = threadIdx.x;
    int hv, c;
    SeqSpan sp;
    if (!block_chunk(p, lane, hv, c, sp)) return;
    const int r = lane & 15, colbase = 4 * (lane >> 4);
    const int t0 = c * BT;
    const bool valid = r < min(BT, sp.len - t0);
    const int64_t tok = sp.tok0 + t0 + r;
    Row32 dop;
    load_row(p.dout + (tok * p.HV + hv) * DK, valid, colbase, dop);
    const i16x4 eye = eye_operand(lane);
    uint8_t* brec = p.ws_bwd + (sp.srec0 + c) * REC_BYTES;
#pragma unroll
    for (int vt = 0; vt < 8; ++vt)
        __builtin_nontemporal_store(__builtin_bit_cast(u32x2, tile_T(dop.v[vt], eye)),
                                    reinterpret_cast<u32x2*>(brec + BREC_DO + vt * 512 + lane * 8));
}

}  // namespace

namespace {
int64_t k1_grid(const Params& p) {
    return p.cu_seqlens ? (int64_t)p.HV * p.NS : (int64_t)p.B * p.HV * p.NT;
}

template <int K1M>
hipError_t launch(const Params& p, hipStream_t stream) {
    const bool all_full = !p.cu_seqlens && p.T % BT == 0;
    auto kern = all_full ? (p.g_bf16 ? k1_kernel<K1M, true, true> : k1_kernel<K1M, true, false>)
                         : (p.g_bf16 ? k1_kernel<K1M, false, true> : k1_kernel<K1M, false, false>);
    hipLaunchKernelGGL(kern, dim3((unsigned)k1_grid(p)), dim3(64), 0, stream, p);
    return hipGetLastError();
}
}  // namespace

hipError_t launch_k1(const Params& p, hipStream_t stream) { return launch<K1_FWD>(p, stream); }

hipError_t launch_k1_both_records(const Params& p, hipStream_t stream) { return launch<K1_BOTH>(p, stream); }

hipError_t launch_k1_save(const Params& p, hipStream_t stream) { return launch<K1_SAVE>(p, stream); }

hipError_t launch_k1_dout(const Params& p, hipStream_t stream) {
    hipLaunchKernelGGL(k1_dout_kernel, dim3((unsigned)k1_grid(p)), dim3(64), 0, stream, p);
    return hipGetLastError();
}

}  // namespace kda
