// Shared device helpers and the chunk-record layout exchanged by the two
// stages of the KDA BT=16 forward on gfx950.
//
// Record layout.  Stage 1 writes one record per (sequence, value head,
// chunk) and stage 2 reads them sequence-head by sequence-head, chunk after
// chunk.  The records of one (sequence, value head) are contiguous:
//   fixed length: record index = (b*HV + hv) * NT + chunk;
//   varlen:       record index = hv * NS + floor(bos_n / 16) + n + chunk,
//                 NS = floor(T / 16) + N (slot map of SeqMap below).
// Every operand is
// stored in the register order in which stage 2 feeds it to the matrix
// cores, so each lane reads its slice with 16-byte loads and no shuffles.
//
// Notation: lane l of a 64-wide wave, r = l & 15 (row inside a 16-lane DPP
// row), q4 = l >> 4 (which of the four 16-lane rows).  A 16-wide column tile
// index is kt (over K) or vt (over V).  "F order" for a 16x128 matrix M
// means lane l holds M[r][16*kt + 4*q4 + i] at item 4*kt + i (kt 0..7,
// i 0..3); "T order" means lane l holds M[4*q4 + i][16*kt + r] at item
// 4*kt + i.
//
//   offset  bytes  content
//   0       4096   w      bf16, F order, stored [j][lane][8]: the 16-byte
//                         operand j (k-tiles 2j, 2j+1) of each lane
//   4096    4096   qg     bf16, F order, [j][lane][8]  = bf16(q^ * 2^G)
//   8192    4096   kg     bf16, T order, [j][lane][8]  = bf16(k^ * 2^(G_last - G))
//   12288    512   Aqk    bf16, [lane][i] = Aqk[r][4*q4+i]
//   12800    512   decay  fp32, [kt][q4][i] = 2^G_last[16*kt+4*q4+i]
//   13312   4096   u      bf16, [vt][lane][i] = u[4*q4+i][16*vt+r]
// The first 13 KiB are read by every value tile of a head, the last 4 KiB
// in 512-byte slices, one per value tile.  Consecutive lanes touch
// consecutive words, so both the global accesses and stage 2's LDS reads
// are conflict free.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kda {

constexpr int BT = 16;    // chunk length (kernels.py:40)
constexpr int DK = 128;   // K == V == 128 (kernels.py:727-728)

constexpr int REC_W = 0;
constexpr int REC_QG = 4096;
constexpr int REC_KG = 8192;
constexpr int REC_AQK = 12288;
constexpr int REC_DECAY = 12800;
constexpr int REC_U = 13312;
constexpr int REC_SHARED = 13312;  // bytes every value tile reads
constexpr int REC_BYTES = 17408;
// Per record slot, what the per-chunk gradient kernel would otherwise
// recompute, exactly as stage 1 formed it (the "gram block", 2 KiB): the
// raw gram Lraw[t][s] = kp_t . km_s (fp32, [lane][i] = Lraw[r][4*q4+i])
// and A_inv = (I + L)^-1 (fp32, [lane][i] = A_inv[r][4*q4+i]).  The
// backward's recompute keeps it in the forward record's qg bytes (qg is not
// needed there: stride REC_BYTES); a training forward that saves its state
// keeps it in a region of its own (stride LA_BYTES).
constexpr int LA_LRAW = 0;
constexpr int LA_AINV = 1024;
constexpr int LA_BYTES = 2048;

// Backward record (kda_bt16_bwd_hip): what the reverse state chain feeds
// its matrix cores, written by the backward's stage-1 pass next to the
// forward record (a second region, same slot indexing).
//   offset  bytes  content
//   0       4096   kg     bf16, F order, [j][lane][8] (k-tiles 2j, 2j+1):
//                         the A operand of dv_new += kg @ dh
//   4096    8192   upd    bf16, [kt][lane][8]: items 0..3 = scale*qg[4*q4+i][16*kt+r]
//                         (bf16(scale * q^ * 2^G)), items 4..7 = -w[4*q4+i][16*kt+r]:
//                         the A operand of dh[kt] += [scale*qg | -w]^T @ [dO ; dv_new]
//   12288   512    AqkT   bf16, [lane][i] = Aqk[4*q4+i][r]: the A operand of Aqk^T @ dO
//   12800   512    decay  fp32, as REC_DECAY
//   13312   4096   dO     bf16, [vt][lane][i] = dO[4*q4+i][16*vt+r]: each value
//                         tile's B operand, where the forward record holds u
// The shared part and the per-tile slices sit where the forward record's
// do, so stage 2's record ring streams either kind unchanged.
constexpr int BREC_KG = 0;
constexpr int BREC_UPD = 4096;
constexpr int BREC_AQKT = 12288;
constexpr int BREC_DECAY = 12800;
constexpr int BREC_DO = 13312;
constexpr int BREC_BYTES = 17408;
static_assert(BREC_BYTES == REC_BYTES && BREC_DECAY == REC_DECAY && BREC_DO == REC_U,
              "backward record has the forward record's shape");

// Training buffers per record slot, bf16, blocked by 16-column value tile
// so that each stage-2 work-group (one value tile) writes whole cache lines:
// the state at the chunk's start h = bf16(S)^T as [vt][k][16] (element
// (k, v) at (v/16 * 128 + k) * 16 + v%16), the gradient of the state after
// the chunk dh likewise, and v_new, dv_new as [vt][row][16] (element
// (row, v) at (v/16 * 16 + row) * 16 + v%16).  Plus per-chunk partial sums
// of the gate-parameter gradients: ddt_bias[128], then dA_log at index 128.
constexpr int TR_H_ELEMS = DK * DK;
constexpr int TR_VN_ELEMS = BT * DK;
constexpr int TR_H_TILE = DK * 16;   // elements of one value tile of h
constexpr int TR_VN_TILE = BT * 16;  // elements of one value tile of v_new
constexpr int PART_STRIDE = 132;

// RCP_LN2 and the l2norm epsilon, kernels.py:38-39.
constexpr float RCP_LN2 = 1.4426950216f;
constexpr float L2_EPS = 1e-6f;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

struct Params {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    const void* g;
    const void* beta;
    const float* A_log;
    const float* dt_bias;
    const float* h0;  // initial state (null: zeros)
    uint16_t* o;
    float* ht;        // final state (null: not stored)
    uint8_t* ws;
    uint16_t* dbg_Aqk;
    uint16_t* dbg_A_inv;
    uint16_t* dbg_w;
    uint16_t* dbg_u;
    float* dbg_g;
    // Value heads: v, g, beta, A_log, dt_bias, the states and o use HV heads,
    // q and k use H, HV a multiple of H (value head hv reads q/k head
    // hv / (HV / H), kernels.py:88).
    int B, T, H, HV, NT;
    // Fixed length: tokens between the first tokens of consecutive batch
    // rows, T for whole rows; a segment of the two-stage forward (launch_two_stage)
    // views tokens [t0, t0 + T) of each row with the row stride kept.
    int64_t tok_stride;
    // Fixed length: chunk c of (row, value head) bh has record slot
    // bh * srec_stride + srec_off + c in the buffers a training forward
    // saves (backward record, gram block, h, v_new), srec_stride 0 meaning
    // NT: a segment of the training forward keeps the whole forward's slots
    // there while its workspace records are the segment's own.
    int srec_stride, srec_off;
    float scale, lower_bound;
    int g_bf16, beta_bf16;
    int use_gate, use_l2norm, use_beta_sigmoid;
    int g_log;  // without use_gate: g is the per-token natural-log decay
    int h0_v_first, ht_v_first;  // layouts of h0 / ht: [V, K] if set, else [K, V]
    int o_fp32;                  // token recurrence only: o in fp32
    // The forward's kernel choices (KdaBt16Args, ABI 4): force_fused /
    // two_stage from the flags; k2_tiles (1, 2, 4, 8) and k2_wave_tiles (1,
    // 2: kda_k2w.hip's compute waves of that many tiles) for stage 2, 0 for
    // the library's choice; max_seqlen, with
    // cu_seqlens, the caller's hint of the longest sequence (0: unknown).
    int force_fused, two_stage;
    int k2_tiles, k2_wave_tiles;
    int max_seqlen;
    // Varlen: N sequences packed along T (B == 1), sequence n holding tokens
    // [cu_seqlens[n], cu_seqlens[n+1]); states are [N, HV, ...].  NS is the
    // number of record slots per value head.  Null cu_seqlens: fixed length.
    const void* cu_seqlens;
    int cu_i64;
    int N, NS;
    // Stage 2 with several sequences (or batch rows) per work-group: the
    // sequences are split into seq_groups contiguous groups (set by
    // launch_k2, 0 for one work-group per sequence).
    int seq_groups;
    // Backward only (kda_bt16_bwd_hip).  Training buffers indexed by record
    // slot (layouts above), the incoming gradients dO [B,T,HV,V] bf16 and
    // dht (state layout of ht, optional), and the outputs: dq, dk, dv bf16 in
    // the shapes of q, k, v; dg and dbeta in the element types of g and beta;
    // dA_log [HV], ddt_bias [HV*128] and dh0 (state layout of h0), each
    // optional as its input is.
    uint8_t* ws_bwd;  // backward records (same slot indexing as ws)
    uint8_t* la;      // gram blocks: slot x at la + x * la_stride
    int64_t la_stride;
    uint16_t* tr_h;
    uint16_t* tr_vn;
    uint16_t* tr_dh;
    uint16_t* tr_dvn;
    float* tr_part;
    const uint16_t* dout;
    const float* dht;
    uint16_t* dq;
    uint16_t* dk;
    uint16_t* dv;
    void* dg;
    void* dbeta;
    float* dA_log;
    float* ddt_bias;
    float* dh0;
};

// Bounds of sequence n of a varlen batch, clamped into [0, T] so that a
// malformed cu_seqlens never leads outside the tensors.
// cu_seqlens is read through the constant address space (it is not
// written while a kernel runs): a uniform index then becomes a scalar load,
// which no vector-memory wait has to cover.
__device__ __forceinline__ int cu_at(const Params& p, int i) {
    typedef __attribute__((address_space(4))) const int64_t c_i64;
    typedef __attribute__((address_space(4))) const int32_t c_i32;
    const int64_t x = p.cu_i64 ? ((c_i64*)p.cu_seqlens)[i] : (int64_t)((c_i32*)p.cu_seqlens)[i];
    return (int)(x < 0 ? 0 : (x > p.T ? p.T : x));
}

// One (sequence or batch row, value head) of the work: its first token in
// the flattened [B*T] token dimension, its length, its chunk count and the
// index of its first record.
struct SeqSpan {
    int64_t tok0;
    int len, nt;
    int64_t rec0;   // first record slot in the workspace
    int64_t srec0;  // first record slot in the saved-state buffers
};

// bh = (batch row or sequence) * HV + hv.
__device__ __forceinline__ SeqSpan seq_span(const Params& p, int bh) {
    SeqSpan s;
    if (p.cu_seqlens) {
        const int n = bh / p.HV, hv = bh - n * p.HV;
        const int bos = cu_at(p, n);
        const int eos = max(bos, cu_at(p, n + 1));
        s.tok0 = bos;
        s.len = eos - bos;
        s.nt = (s.len + BT - 1) / BT;
        s.rec0 = (int64_t)hv * p.NS + bos / BT + n;
        s.srec0 = s.rec0;
    } else {
        s.tok0 = (int64_t)(bh / p.HV) * p.tok_stride;
        s.len = p.T;
        s.nt = p.NT;
        s.rec0 = (int64_t)bh * p.NT;
        s.srec0 = (int64_t)bh * (p.srec_stride ? p.srec_stride : p.NT) + p.srec_off;
    }
    return s;
}

// Stands in for an optional per-column operand (dt_bias, A_log) that is
// absent, so that its loads stay unconditional (a pointer select, not a
// branch).  Never written.  Global memory, not constant, so that the
// selected pointer stays a global one and its loads are counted in order
// with the others by the wait counters.  One copy per source file.
namespace {
__device__ __attribute__((visibility("hidden"))) float kZeroCols[DK];
}

// Varlen: the sequence n whose record slots hold slot x, i.e. the largest n
// with floor(cu_seqlens[n] / 16) + n <= x (strictly increasing in n for a
// non-decreasing cu_seqlens).  A 64-way search: each round every lane tests
// one candidate and the ballot's population count is the number of
// candidates at or below x.  Any cu_seqlens gives an n in [0, N).
__device__ __forceinline__ int find_sequence(const Params& p, int x, int lane) {
    int lo = 0, cnt = p.N;
    while (cnt > 1) {
        const int step = (cnt + 63) >> 6;
        const int idx = lo + lane * step;
        const bool below = idx < lo + cnt && cu_at(p, idx) / BT + idx <= x;
        const int m = __popcll(__ballot(below));
        if (m == 0) break;
        const int next = lo + (m - 1) * step;
        cnt = min(step, lo + cnt - next);
        lo = next;
    }
    return lo;
}

// bf16 <-> fp32.  fp32 -> bf16 rounds to nearest even (the hardware
// conversion on gfx950), matching torch's .to(torch.bfloat16).
__device__ __forceinline__ float bf2f(uint16_t h) {
    return __builtin_bit_cast(float, (uint32_t)h << 16);
}
__device__ __forceinline__ uint16_t f2bf(float x) {
    return __builtin_bit_cast(uint16_t, (__bf16)x);
}
// Round a float to the nearest bf16 value and return it as float.
__device__ __forceinline__ float round_bf(float x) { return bf2f(f2bf(x)); }

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two floats to two bf16 (round to nearest even) in one v_cvt_pk_bf16_f32;
// `a` lands in the low half.
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

// exp2 on the transcendental unit (v_exp_f32, 1 ulp), without the library
// routine's denormal-range fixups: every exponent that reaches it is either
// in the normal range or so negative that the result is a negligible
// underflow, as with Triton's exp2 on GPUs.
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// sigmoid(x) = 1 / (1 + e^-x) with v_exp_f32 and v_rcp_f32 (~2 ulp).
// Saturates correctly: x -> -inf gives rcp(inf) = 0, x -> +inf gives 1.
__device__ __forceinline__ float fast_sigmoid(float x) {
    return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}

// Inclusive prefix sum over the 16 lanes of a DPP row (row_shr:1,2,4,8).
// Lanes shifted in from outside the row contribute 0.
__device__ __forceinline__ float row_scan16(float x) {
#define KDA_SCAN_STEP(n)                                                      \
    x += __builtin_bit_cast(                                                  \
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x),     \
                                           0x110 + (n), 0xf, 0xf, false));
    KDA_SCAN_STEP(1)
    KDA_SCAN_STEP(2)
    KDA_SCAN_STEP(4)
    KDA_SCAN_STEP(8)
#undef KDA_SCAN_STEP
    return x;
}

// Lane LANE of each 16-lane row to the whole row (DPP row_newbcast).
template <int LANE>
__device__ __forceinline__ float row_bcast(float v) {
    constexpr int ROW_NEWBCAST = 0x150;
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                 ROW_NEWBCAST + LANE, 0xf, 0xf,
                                                                 false));
}

// Sum over each 16-lane row, every lane receiving it, by DPP: quad_perm
// pairs lanes 1 and 2 apart, then row_half_mirror pairs the two quads of
// each half-row and row_mirror the two half-rows.  After each step the
// lanes of a group hold the same value, so the last two steps add what
// lane ^ 4 and lane ^ 8 would: the bits of the shuffle tree over 1, 2, 4, 8.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xf, 0xf, true));
}
__device__ __forceinline__ float row_sum16(float x) {
    constexpr int QP_XOR1 = 0xB1;  // quad_perm [1,0,3,2]
    constexpr int QP_XOR2 = 0x4E;  // quad_perm [2,3,0,1]
    constexpr int ROW_HALF_MIRROR = 0x141;
    constexpr int ROW_MIRROR = 0x140;
    x += dpp_mov<QP_XOR1>(x);
    x += dpp_mov<QP_XOR2>(x);
    x += dpp_mov<ROW_HALF_MIRROR>(x);
    x += dpp_mov<ROW_MIRROR>(x);
    return x;
}

// The value of lane ^ 16 (within each 32 lanes), by ds_swizzle in bit mode:
// and_mask 0x1f, or_mask 0, xor_mask 0x10.
__device__ __forceinline__ float xor16(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, x), 0x401F));
}

__device__ __forceinline__ float shfl(float x, int src_lane) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_ds_bpermute(src_lane << 2, __builtin_bit_cast(int, x)));
}

// Matrix-core wrappers (gfx950).  Operand/result layouts for the 16x16
// shapes: A[m][k] comes from lane m + 16*(k / kpl) item k % kpl, B[k][n]
// from lane n + 16*(k / kpl) item k % kpl, and D[m][n] lands in lane
// n + 16*(m / 4) item m % 4, with kpl = 1, 4, 8 for K = 4, 16, 32.
__device__ __forceinline__ f32x4 mfma_f32_16x16x4(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_bf16_16x16x16(i16x4 a, i16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_bf16_16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// A 16x16x16 product (4 bf16 of k per lane) issued as a 16x16x32 one whose
// k items 4..7 are zero in both operands: the same sum of products, for a
// chain of accumulating 16x16x32 MFMAs.  On gfx950 an MFMA that accumulates
// (SrcC = its vdst) onto the result of an MFMA of the other shape
// (16x16x16 <-> 16x16x32) fewer than 5 wait states later reads stale
// values for two of its four accumulator registers (items 2-3 after a
// 16x16x16, 0-1 after a 16x16x32; measured over 10^6 trials each), and the
// compiler puts no wait state between such a pair.  One shape per chain
// avoids the case: back-to-back accumulation of one shape forwards
// correctly.  tests/test_mfma_hazards.py checks the built library for
// mixed-shape accumulation closer than 8 wait states.
__device__ __forceinline__ f32x4 mfma_bf16_16x16x16_in_x32(u32x2 a, u32x2 b, f32x4 c) {
    return mfma_bf16_16x16x32(__builtin_bit_cast(bf16x8, u32x4{a.x, a.y, 0u, 0u}),
                              __builtin_bit_cast(bf16x8, u32x4{b.x, b.y, 0u, 0u}), c);
}

__device__ __forceinline__ i16x4 as_i16x4(u32x2 v) { return __builtin_bit_cast(i16x4, v); }

// 4x4 transpose of 16-bit values across the 4 lanes of a quad.  Lane j
// enters with p0 = (M[0][j], M[1][j]) and p1 = (M[2][j], M[3][j]) and leaves
// with (M[j][0], M[j][1]) and (M[j][2], M[j][3]).  Two DPP exchanges:
// lanes j and j^2 swap the 2x2 blocks off the diagonal, then lanes j and
// j^1 swap 16-bit halves.  Applied to a 16x16 accumulator tile (lane
// (x, q4) holding rows 4*q4 .. +3 of column x), it leaves lane (x, q4) with
// row 4*q4 + x%4, columns 4*(x/4) .. +3: one 8-byte row-major store per
// lane.  Applied to such row pieces, it gives back the tile layout.
__device__ __forceinline__ u32x2 quad_transpose(uint32_t p0, uint32_t p1, int j) {
    constexpr int QP_XOR2 = 2 | (3 << 2) | (0 << 4) | (1 << 6);  // quad_perm [2,3,0,1]
    constexpr int QP_XOR1 = 1 | (0 << 2) | (3 << 4) | (2 << 6);  // quad_perm [1,0,3,2]
    const bool lo2 = (j & 2) == 0;
    // after this, the lane holds rows {r, r+1} (r = 0 for j < 2, else 2)
    // for columns {j & 1, (j & 1) + 2} as (a: column j&1, b: column (j&1)+2)
    const uint32_t send2 = lo2 ? p1 : p0;
    const uint32_t recv2 = (uint32_t)__builtin_amdgcn_mov_dpp((int)send2, QP_XOR2, 0xf, 0xf, false);
    const uint32_t a = lo2 ? p0 : recv2;
    const uint32_t bb = lo2 ? recv2 : p1;
    // lane with j even keeps the low halves (its row), sends the high halves
    const bool even = (j & 1) == 0;
    const uint32_t send1 = even ? __builtin_amdgcn_perm(bb, a, 0x07060302u)   // (a.hi, b.hi)
                                : __builtin_amdgcn_perm(bb, a, 0x05040100u);  // (a.lo, b.lo)
    const uint32_t recv1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)send1, QP_XOR1, 0xf, 0xf, false);
    // even lane: (a.lo, recv.lo), (b.lo, recv.hi); odd lane: (recv.lo, a.hi), (recv.hi, b.hi)
    const uint32_t w0 = even ? __builtin_amdgcn_perm(recv1, a, 0x05040100u)
                             : __builtin_amdgcn_perm(a, recv1, 0x07060100u);
    const uint32_t w1 = even ? __builtin_amdgcn_perm(recv1, bb, 0x07060100u)
                             : __builtin_amdgcn_perm(bb, recv1, 0x07060302u);
    return u32x2{w0, w1};
}
__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

}  // namespace kda

// Host-side launchers (defined next to each kernel).
namespace kda {
hipError_t launch_k1(const Params& p, hipStream_t stream);
hipError_t launch_k2(const Params& p, hipStream_t stream);
// Stage 2 with several value tiles per work-group (kda_k2w.hip): the tile
// count launch_k2 picks for a geometry on `ncu` CUs (0: one per work-group),
// and the launch with `tpw` tiles (2, 4 or 8).
int k2_wide_tiles(const Params& p, int ncu);
hipError_t launch_k2_wide(const Params& p, int tpw, hipStream_t stream);
// The forward as one kernel (kda_fused.hip): whether it is taken for a
// geometry on `ncu` CUs, its launch, and the count of its work-groups that
// gave up a bounded wait on the current device (read synchronously, then
// optionally reset).
bool fused_forward(const Params& p, int ncu);
hipError_t launch_fused(const Params& p, hipStream_t stream);
hipError_t fused_abort_count(uint32_t* count, bool reset);
// The forward is fused or stage 1 then stage 2 (kda_k2.hip); fwd_plan says
// which on the current device (1 fused, 0 two stages), and fwd_segments in
// how many segments of consecutive chunks the two stages run.
int fwd_plan(const Params& p);
int fwd_segments(const Params& p);
hipError_t launch_two_stage(const Params& p, hipStream_t stream);
hipError_t launch_fwd_save(const Params& p, hipStream_t stream);
int64_t segment_bytes(const Params& p, int nseg);
int segments_to_fit(const Params& p, int64_t max_bytes);
hipError_t launch_two_stage_in(const Params& p, int nseg, hipStream_t stream);
hipError_t launch_recurrent(const Params& p, hipStream_t stream);
// Backward (kda_bt16_bwd.hip, and the training variants of the stages).
hipError_t launch_k1_both_records(const Params& p, hipStream_t stream);
hipError_t launch_k2_train(const Params& p, hipStream_t stream);
// Training forward that saves its state for the backward, and the
// backward's completion of the saved backward records with dO.
hipError_t launch_k1_save(const Params& p, hipStream_t stream);
hipError_t launch_k2_train_o(const Params& p, hipStream_t stream);
hipError_t launch_k1_dout(const Params& p, hipStream_t stream);
hipError_t launch_k2_bwd(const Params& p, hipStream_t stream);
hipError_t launch_bwd_chunk(const Params& p, hipStream_t stream);
hipError_t launch_bwd_gate_reduce(const Params& p, hipStream_t stream);
}  // namespace kda
