// The KDA BT=16 forward in one kernel, for shapes with more (sequence, head)
// pairs than half the CUs (batched and varlen prefill).
//
// The two-stage forward (kda_k1.hip, then kda_k2.hip / kda_k2w.hip) passes
// each chunk's 17 KiB record through HBM: written by stage 1, read back by
// stage 2.  Once the (sequence, head) pairs fill the CUs that round trip is
// most of the forward's traffic (B=16 T=2048 H=32: 3.7 GB moved per forward
// for 1.4 GB of inputs and outputs).  Here one work-group per (sequence,
// value head) keeps the records in LDS:
//   * NP producer waves each form every NP-th chunk's record with stage 1's
//     per-chunk code (k1_compute, kda_k1_chunk.h) straight into a ring of
//     RING record slots in LDS, each with its own LDS scratch; each loads
//     its next chunk's q, k and g rows into an LDS staging area while it
//     works on the current one;
//   * four compute waves each run the recurrence for two of the head's
//     eight 16-column value tiles (wide_step, kda_k2w_step.h), reading the
//     operands every tile shares from the slot.
// The arithmetic is stage 1's and the wide stage 2's, so o and ht are bit
// for bit those of the two-stage forward.
//
// The waves meet through LDS words, never at a barrier after the start
// (a barrier would hold the compute waves' steps to the producers' chunks):
//   full[s]  = c + 1 once chunk c's record is complete in slot s = c % RING
//              (the producer's LDS writes have completed before it stores it);
//   done[s]  counts the compute waves' reads of slot s, NCW per chunk: the
//              producer of chunk c waits for NCW * (c / RING) before writing
//              slot s, that is until chunk c - RING has been read by all.
// Chunk c's producer only waits for reads of chunk c - RING, which needs
// only chunks below c, all produced by then (each producer takes its chunks
// in order), so the waits always end.  Each wait is also bounded (SPIN_LIMIT
// polls) so that a stalled work-group cannot hang the GPU: a bound that runs
// out marks the work-group aborted, after which no wave waits again; the
// work-group drains, its compute waves that had not finished write NaN over
// their o columns and final-state rows, and it adds 1 to a device-wide
// count that the host reads (fused_abort_count).
#include "kda_common.h"
#include "kda_k1_chunk.h"
#include "kda_k2_shared.h"
#include "kda_k2w_step.h"

namespace kda {

namespace {

constexpr int F_NCW = 4;  // compute waves, two value tiles each
constexpr int F_NP = 4;   // producer waves
constexpr int F_RING = 4; // record slots
constexpr int F_THREADS = 64 * (F_NCW + F_NP);
constexpr int SPIN_LIMIT = 1 << 22;
static_assert(F_RING >= F_NP, "every producer can hold a slot");

// A producer's staging area for the next chunk's q, k and g rows, which it
// loads straight into LDS (direct buffer->LDS loads) while it works on the
// current chunk: 16 rows of 256 bytes for q and k, of 256 (bf16) or 512
// (fp32) bytes for g.
constexpr int ST_Q = 0, ST_K = 4096, ST_G = 8192, STAGE_BYTES = 16384;

// The work-group's LDS.
__shared__ __attribute__((aligned(1024))) uint8_t f_ring[F_RING][FREC_BYTES];
__shared__ __attribute__((aligned(1024))) uint8_t f_stage[F_NP][STAGE_BYTES];
__shared__ __attribute__((aligned(16))) uint8_t f_scratch[F_NP][K1_SCRATCH];
__shared__ __attribute__((aligned(16))) float f_bias[DK];  // the head's dt_bias (zeros without it)
__shared__ int f_full[F_RING];
__shared__ int f_done[F_RING];
__shared__ int f_aborted;
__shared__ int f_counted;  // the work-group's give-up has been counted

// Work-groups that gave up a wait on this device since the library was
// loaded or the count was reset (fused_abort_count).
__device__ uint32_t g_aborts;

__device__ __forceinline__ int lds_load(const int* a) {
    return __builtin_amdgcn_readfirstlane(__hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
}

// Polls the LDS word `a` until it reaches `target` (bounded; see above).
__device__ __forceinline__ void wait_ge(const int* a, int target) {
    for (int i = 0; i < SPIN_LIMIT; ++i) {
        if (lds_load(a) >= target || lds_load(&f_aborted)) {
            asm volatile("" ::: "memory");
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    __hip_atomic_store(&f_aborted, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    asm volatile("" ::: "memory");
}

// A work-group that gave up a wait has read slots whose chunks it cannot
// vouch for: this compute wave's o columns (its two value tiles) over the
// whole sequence and its final-state rows become NaN.
__device__ __forceinline__ void mark_lost(const Params& p, const SeqSpan& sp, int hv, int ut, int lane,
                                       f32x4 (&SA)[8], f32x4 (&SB)[8]) {
    const float nan = __builtin_nanf("");
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
        SA[kt] = f32x4{nan, nan, nan, nan};
        SB[kt] = SA[kt];
    }
    // the wave's o stores of the chunks have completed before these replace them
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    const u32x4 nan8 = {0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u};
    uint16_t* base = p.o + (sp.tok0 * p.HV + hv) * DK + 16 * ut + 8 * (lane & 3);
    for (int r = lane >> 2; r < sp.len; r += 16)
        *reinterpret_cast<u32x4*>(base + (int64_t)r * p.HV * DK) = nan8;
}

// The compute waves' side of the LDS flags (wide_step's hooks), and their
// share of stage 1: u of their two tiles, formed from the raw v tiles,
// bf16(A_inv) and beta the producers leave in u's place (FREC_*), with the
// instructions stage 1 uses (form_u).  The producers pace the work-group;
// this moves ~6 % of their issue work to the compute waves, which wait for
// them most of the time.
template <int S>
struct FlagHooks {
    u32x2 v[2], a;  // raw v of the two tiles, bf16(A_inv) as the A operand
    float beta;     // beta of this lane's row
    __device__ __forceinline__ void ready(int c) { wait_ge(&f_full[S], c + 1); }
    __device__ __forceinline__ void read_u(const uint8_t* slot, int lane, int ut) {
        v[0] = *reinterpret_cast<const u32x2*>(slot + REC_U + ut * 512 + lane * 8);
        v[1] = *reinterpret_cast<const u32x2*>(slot + REC_U + (ut + 1) * 512 + lane * 8);
        a = *reinterpret_cast<const u32x2*>(slot + FREC_A + lane * 8);
        beta = *reinterpret_cast<const float*>(slot + FREC_BETA + 4 * (lane & 15));
    }
    __device__ __forceinline__ f32x4 u_start(int t) const {
        const int lane = threadIdx.x & 63;
        return unpack_u(form_u(v[t], beta, as_i16x4(a), eye_operand(lane)));
    }
    __device__ __forceinline__ void consumed() {
        // the slot reads have completed before they are counted
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if ((threadIdx.x & 63) == 0)
            __hip_atomic_fetch_add(&f_done[S], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    __device__ __forceinline__ void end() {}
};

// Chunks c .. c + N - 1 (those below NT) from slot S on.
template <int S, int N>
__device__ __forceinline__ void fused_round(const WideCtx& cx, int c, f32x4 (&SA)[8], f32x4 (&SB)[8],
                                            int ut) {
    if (c >= cx.NT) return;
    FlagHooks<S> hk;
    wide_step(cx, c, SA, SB, f_ring[S], ut, hk);
    if constexpr (N > 1) fused_round<(S + 1) % F_RING, N - 1>(cx, c + 1, SA, SB, ut);
}

// The LDS address of an LDS pointer (wave-uniform).
__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_u8*)p);
}

// A raw buffer descriptor over `bytes` bytes from `base`, in SGPRs.
typedef int i32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ i32x4 buffer_words(const void* base, uint32_t bytes) {
    const uint64_t a = reinterpret_cast<uintptr_t>(base);
    return i32x4{__builtin_amdgcn_readfirstlane((int)(uint32_t)a),
                 __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffffu)),
                 __builtin_amdgcn_readfirstlane((int)bytes), BUF_DWORD3};
}

// One direct buffer->LDS load of 16 bytes a lane (lane l's to LDS address
// lds + 16 l).  Written as inline asm so that the compiler, which cannot
// tell which LDS bytes such a load writes, does not wait for it before every
// later LDS access of the wave; the producer waits for it itself (vmcnt)
// before it reads the staging area.  The load takes its LDS address from
// M0, which the block saves and restores (the compiler may hold a value
// there); a wait state separates each M0 write from the next use, as the
// compiler's own direct loads have.
__device__ __forceinline__ void dma16(i32x4 rs, uint32_t lds, uint32_t voff) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "s_nop 0\n\t"
        "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0"
        : "=&s"(saved) : "s"(lds), "v"(voff), "s"(rs) : "memory");
}

// Staging layout: 16 rows of UNITS 16-byte units (16 for a bf16 row, 32
// for an fp32 row); unit u of row r sits at position r * UNITS +
// (u + r) % UNITS, so that the 16 lanes reading one unit column of the 16
// rows hit 16 different bank groups.  One direct load moves 64 units (lane
// l to position 64 i + l); rows past the sequence's end lie outside the
// buffer descriptor's range, are not read, and are zeroed when read back.
template <int UNITS>
__device__ __forceinline__ void stage_issue(i32x4 rs, uint32_t dst, int lane, uint32_t row_stride) {
#pragma unroll
    for (int i = 0; i < UNITS / 4; ++i) {
        const int pos = 64 * i + lane;
        const int r = pos / UNITS;
        const int u = (pos - r) & (UNITS - 1);
        dma16(rs, dst + i * 1024, r * row_stride + u * 16);
    }
}

// The direct loads of chunk c's q, k and g rows into the staging area at
// LDS address st.
template <bool GB16>
__device__ __forceinline__ void stage_chunk(const Params& p, int hv, int c, const SeqSpan& sp, uint32_t st,
                                            int lane) {
    const int h = hv / (p.HV / p.H);
    const int nvalid = min(BT, sp.len - c * BT);
    const int64_t tok = sp.tok0 + c * BT;
    const uint32_t qs = (uint32_t)p.H * DK * 2, gs = (uint32_t)p.HV * DK * (GB16 ? 2 : 4);
    const i32x4 rq = buffer_words(p.q + (tok * p.H + h) * DK, nvalid * qs);
    const i32x4 rk = buffer_words(p.k + (tok * p.H + h) * DK, nvalid * qs);
    const i32x4 rg = buffer_words(static_cast<const uint8_t*>(p.g) + (tok * p.HV + hv) * DK * (GB16 ? 2 : 4),
                                  nvalid * gs);
    stage_issue<16>(rq, st + ST_Q, lane, qs);
    stage_issue<16>(rk, st + ST_K, lane, qs);
    stage_issue<GB16 ? 16 : 32>(rg, st + ST_G, lane, gs);
}

// This lane's q, k and g values of the staged chunk, in k1_load's layout.
template <bool FULL, bool GB16>
__device__ __forceinline__ void stage_read(const uint8_t* st, int lane, bool valid, K1In<GB16, false>& in) {
    const int r = lane & 15, q4 = lane >> 4;
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
        const int b16 = (r * 16 + ((2 * kt + (q4 >> 1) + r) & 15)) * 16 + (q4 & 1) * 8;
        in.q.v[kt] = *reinterpret_cast<const u32x2*>(st + ST_Q + b16);
        in.k.v[kt] = *reinterpret_cast<const u32x2*>(st + ST_K + b16);
        if constexpr (GB16) {
            in.g16.v[kt] = *reinterpret_cast<const u32x2*>(st + ST_G + b16);
        } else {
            in.g32[kt] = *reinterpret_cast<const f32x4*>(st + ST_G + (r * 32 + ((4 * kt + q4 + r) & 31)) * 16);
        }
        if (!FULL && !valid) {
            in.q.v[kt] = u32x2{0u, 0u};
            in.k.v[kt] = u32x2{0u, 0u};
            in.g16.v[kt] = u32x2{0u, 0u};
            in.g32[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
}

// beta of this lane's row of chunk c (raw bits; 0 past the sequence's end).
__device__ __forceinline__ uint32_t load_beta(const Params& p, int hv, int c, const SeqSpan& sp, int lane) {
    const int r = lane & 15;
    if (c * BT + r >= sp.len) return 0u;
    const int64_t bi = (sp.tok0 + c * BT + r) * p.HV + hv;
    return p.beta_bf16 ? static_cast<const uint16_t*>(p.beta)[bi] : static_cast<const uint32_t*>(p.beta)[bi];
}

// One chunk of a producer: its staged inputs to registers, v straight from
// HBM (first used late in the chunk), the next chunk's staging and beta
// issued, then stage 1's work into the ring slot.  `beta` holds this chunk's
// beta on entry and the next chunk's on return.
template <bool FULL, bool GB16>
__device__ __forceinline__ void produce(const Params& p, int hv, int c, int c_next, const SeqSpan& sp,
                                        uint8_t* st, uint8_t* scr, float ea, uint32_t& beta, int lane) {
    K1In<GB16, false> in;
    const K1Row w = k1_row<FULL>(p, hv, c, sp);
    // the staged rows of chunk c have landed (only direct loads are in flight)
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    stage_read<FULL, GB16>(st, lane, w.valid, in);
    load_row(p.v + w.vrowoff, w.valid, w.colbase, in.v);
    in.beta_bits = beta;
    // the staging area is read before it is overwritten
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (c_next < sp.nt) {
        stage_chunk<GB16>(p, hv, c_next, sp, lds_addr(st), lane);
        beta = load_beta(p, hv, c_next, sp, lane);
    }
    const int s = c % F_RING;
    wait_ge(&f_done[s], F_NCW * (c / F_RING));
    float* sL = reinterpret_cast<float*>(scr);
    float* sX = reinterpret_cast<float*>(scr + K1_SCRATCH_L);
    k1_compute<K1_FWD, FULL, GB16, true>(p, hv, c, sp, in, f_bias, ea, sL, sX, f_ring[s]);
    // the record's LDS writes have completed before the slot is marked full
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (lane == 0) __hip_atomic_store(&f_full[s], c + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Producer wave pw: chunks pw, pw + NP, ... of the sequence, each into its
// slot once the slot's previous chunk has been read by every compute wave.
// The q, k and g rows of its next chunk load into its staging area while it
// works on this one, so their HBM round trip overlaps that work.
template <bool GB16>
__device__ __forceinline__ void producer_wave(const Params& p, int pw, int hv, const SeqSpan& sp) {
    const int lane = threadIdx.x & 63;
    uint8_t* st = f_stage[pw];
    uint8_t* scr = f_scratch[pw];
    const float ea = k1_ea(p, hv);
    if (pw >= sp.nt) return;
    stage_chunk<GB16>(p, hv, pw, sp, lds_addr(st), lane);
    uint32_t beta = load_beta(p, hv, pw, sp, lane);
    for (int c = pw; c < sp.nt; c += F_NP) {
        if ((c + 1) * BT <= sp.len) {
            produce<true, GB16>(p, hv, c, c + F_NP, sp, st, scr, ea, beta, lane);
        } else {
            produce<false, GB16>(p, hv, c, c + F_NP, sp, st, scr, ea, beta, lane);
        }
    }
}

// The (sequence or batch row, value head) of work-group wg.  A work-group
// runs as long as its sequence, and work-groups start in id order as CUs
// free up: with cu_seqlens (up to 64 sequences) the ids go to the sequences
// longest first, each sequence's heads together, so that the longest chains
// start at once and the short ones fill in around them.  Otherwise the
// natural order.
__device__ __forceinline__ int fused_pair(const Params& p, int wg) {
    if (!p.cu_seqlens || p.N > 64) return wg;
    const int lane = threadIdx.x & 63;
    const int len = lane < p.N ? cu_at(p, lane + 1) - cu_at(p, lane) : -1;
    // rank of this lane's sequence: the sequences longer, or as long with a
    // lower index
    int rank = 0;
    for (int m = 0; m < p.N; ++m) {
        const int lm = __builtin_amdgcn_readlane(len, m);
        rank += (lm > len || (lm == len && m < lane)) ? 1 : 0;
    }
    const int s = wg / p.HV;
    const uint64_t hit = __ballot(lane < p.N && rank == s);
    if (hit == 0) return wg;  // (the ranks are a permutation: never taken)
    const int n = __builtin_amdgcn_readfirstlane((int)__builtin_ctzll(hit));
    return n * p.HV + (wg - s * p.HV);
}

// One work-group per (sequence or batch row, value head).
template <bool GB16>
__global__ __launch_bounds__(F_THREADS) void fused_kernel(Params p) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int bh = fused_pair(p, blockIdx.x);
    const int hv = bh - (bh / p.HV) * p.HV;
    const SeqSpan sp = seq_span(p, bh);
    const int64_t sbase = (int64_t)bh * DK * DK;
    const int q4 = lane >> 4;

    if (sp.nt == 0) {
        // an empty sequence: its final state is its initial state (no wave
        // reaches the barrier below)
        if (wave < F_NCW) {
            f32x4 St[8];
            for (int t = 0; t < 2; ++t) {
                const int v = 16 * (2 * wave + t) + (lane & 15);
                load_state(p, sbase, v, q4, St);
                store_state(p, sbase, v, q4, St);
            }
        }
        __builtin_amdgcn_endpgm();
    }
    if (threadIdx.x < F_RING) {
        f_full[threadIdx.x] = 0;
        f_done[threadIdx.x] = 0;
    }
    if (threadIdx.x == 0) {
        f_aborted = 0;
        f_counted = 0;
    }
    if (threadIdx.x < DK) f_bias[threadIdx.x] = p.use_gate && p.dt_bias ? p.dt_bias[hv * DK + threadIdx.x] : 0.f;
    __syncthreads();

    if (wave >= F_NCW) {
        // The producers pace the work-group (B=16 T=2048 H=32: the compute
        // waves' work alone takes 270 us, the producers' alone 900): on the
        // SIMD a producer shares with a compute wave it issues first
        // (649 -> 605 us).
        __builtin_amdgcn_s_setprio(1);
        producer_wave<GB16>(p, wave - F_NCW, hv, sp);
        __builtin_amdgcn_endpgm();
    }
    const int ut = 2 * wave;                // this wave's first value tile
    const int va = 16 * ut + (lane & 15);   // this lane's state row of it
    f32x4 SA[8], SB[8];
    load_state(p, sbase, va, q4, SA);
    load_state(p, sbase, va + 16, q4, SB);
    WideCtx cx;
    cx.scale = p.scale;
    cx.NT = sp.nt;
    cx.T = sp.len;
    cx.lane = lane;
    cx.q4 = q4;
    cx.obase[0] = p.o + (sp.tok0 * p.HV + hv) * DK + 16 * ut + 4 * ((lane & 15) >> 2);
    cx.obase[1] = cx.obase[0] + 16;
    cx.orow_stride = (int64_t)p.HV * DK;
    for (int c = 0; c < cx.NT; c += F_RING) fused_round<0, F_RING>(cx, c, SA, SB, ut);
    // Every give-up is seen here by at least one compute wave: a producer
    // marks the work-group before it publishes the chunk it gave up on, and
    // this wave consumed every chunk; a compute wave sees its own.  The first
    // compute wave to see it counts the work-group, outside every wait loop.
    if (lds_load(&f_aborted)) {
        if (lane == 0 &&
            __hip_atomic_exchange(&f_counted, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) == 0)
            __hip_atomic_fetch_add(&g_aborts, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        mark_lost(p, sp, hv, ut, lane, SA, SB);
    }
    store_state(p, sbase, va, q4, SA);
    store_state(p, sbase, va + 16, q4, SB);
    __builtin_amdgcn_endpgm();
}

}  // namespace

// Estimated times (us) of a varlen forward on `ncu` CUs, from per-chunk
// costs measured on MI355X (K = V = 128, every in-kernel flag):
//   fused: each work-group takes ~1.85 us per chunk of its sequence, in
//     parallel with the others, so the longest sequence sets the time, or
//     the chunks per CU once the work-groups run in rounds;
//   two stages: stage 1 ~7.5 ns per record slot and value head, stage 2
//     ~0.65 us per step of its longest chain (or of the chunks per CU).
// Measured at 192 (sequence, head) pairs (HV = 32): lengths 19456 + 5 x
// 1024, fused 2188 us and two stages 1146 (estimates 2250 and 1160);
// 6 x 4096, 480 against 590 (474 and 536).
double fused_estimate_us(const Params& p, int ncu) {
    const double chunks = (double)((std::min(p.max_seqlen, p.T) + BT - 1) / BT);
    const double per_cu = (double)p.HV * p.NS / ncu;
    return 1.85 * std::max(chunks, per_cu);
}

double two_stage_estimate_us(const Params& p, int ncu) {
    const double chunks = (double)((std::min(p.max_seqlen, p.T) + BT - 1) / BT);
    const double slots = (double)p.HV * p.NS;
    return 0.0075 * slots + 0.65 * std::max(chunks, slots / ncu);
}

// Whether the forward runs as one fused kernel: never when the
// reference-layout intermediates are asked for (those come from stage 1);
// as the caller asks (force_fused, the reference's use_fused_kernel, or
// two_stage); else, with fixed length, when the (sequence, head) pairs are
// more than half the CUs; with cu_seqlens and the caller's max_seqlen, when
// the fused estimate is at most the two stages'; with cu_seqlens alone,
// when the pairs fill the CUs.
//
// Below the CU count the fused kernel runs every pair in one round of
// work-groups, about 1.85 us per chunk whatever their number, while the two
// stages grow with the pairs (T=4096 forwards, two stages against fused: 128
// pairs 377 against 476 us, 160 pairs 505 against 480, 224 pairs 658 against
// 479).  With cu_seqlens the fused kernel's time follows the longest
// sequence and stage 1's the total: a single long sequence among short ones
// makes the fused kernel up to about twice slower (192 pairs, lengths
// 19456 + 5 x 1024: fused 2188 us, two stages 1146; equal lengths: 480
// against 590).  Without the length of the longest sequence, the pairs
// must fill the CUs.
bool fused_forward(const Params& p, int ncu) {
    if (p.dbg_w || p.dbg_u || p.dbg_Aqk || p.dbg_A_inv || p.dbg_g) return false;
    if (p.force_fused) return true;
    if (p.two_stage) return false;
    const int64_t nbh = (int64_t)(p.cu_seqlens ? p.N : p.B) * p.HV;
    if (!p.cu_seqlens) return 2 * nbh > ncu;
    if (p.max_seqlen > 0) return fused_estimate_us(p, ncu) <= two_stage_estimate_us(p, ncu);
    return nbh >= ncu;
}

hipError_t launch_fused(const Params& p, hipStream_t stream) {
    const int64_t nbh = (int64_t)(p.cu_seqlens ? p.N : p.B) * p.HV;
    auto kern = p.g_bf16 ? fused_kernel<true> : fused_kernel<false>;
    hipLaunchKernelGGL(kern, dim3((unsigned)nbh), dim3(F_THREADS), 0, stream, p);
    return hipGetLastError();
}

hipError_t fused_abort_count(uint32_t* count, bool reset) {
    hipError_t e = hipDeviceSynchronize();
    if (e != hipSuccess) return e;
    e = hipMemcpyFromSymbol(count, HIP_SYMBOL(g_aborts), sizeof(uint32_t), 0, hipMemcpyDeviceToHost);
    if (e != hipSuccess || !reset) return e;
    const uint32_t zero = 0;
    return hipMemcpyToSymbol(HIP_SYMBOL(g_aborts), &zero, sizeof(uint32_t), 0, hipMemcpyHostToDevice);
}

}  // namespace kda
