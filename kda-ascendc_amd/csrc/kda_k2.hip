// Stage 2 of the KDA BT=16 forward: the serial delta-rule recurrence.
//
// Follows kda_bt16_kernel_k2 (/root/reference/src/kda_bt16/kernels.py:187-302):
// per chunk,
//   hc    = bf16(S)
//   v_new = bf16(u - w @ hc^T)
//   o     = bf16(scale * (qg @ hc^T) + Aqk @ v_new)
//   S     = S * 2^G_last[None, :] + (kg^T @ v_new)^T
// with S the [V, K] fp32 state.
//
// One work-group of three waves per (batch, head, 16 value columns), each
// wave on its own SIMD:
//   * the state wave runs the recurrence.  It keeps its slice of S
//     transposed, S^T[k][v], as eight 16x16 fp32 accumulator tiles; the
//     16x16 accumulator layout (lane v + 16*(k/4), item k%4) is exactly the
//     B-operand layout of the 16x16x16 bf16 matrix op, so bf16(S) feeds the
//     next chunk's products straight from registers.  Pairs of k-tiles form
//     the 8-deep operands of the 16x16x32 op for w @ hc^T; stage 1 stored w
//     and qg in the matching k order.  It reads the next chunk's operands
//     while it computes this one, and hands hc and v_new to the output wave.
//   * the output wave forms o two chunks behind, from hc, v_new, qg and Aqk,
//     and stores it.
//   * the copy wave streams the chunk records from HBM into an LDS ring
//     ahead of use (gfx950 direct buffer->LDS loads).
// The three meet at one barrier per chunk.  Only the copy wave waits on
// loads and only the output wave stores, so neither memory latency sits on
// the state wave's chain.
#include <algorithm>
#include <type_traits>

#include "kda_common.h"
#include "kda_k2_shared.h"

namespace kda {

namespace {

// Record ring: RING slots, each the 13 KiB every value tile needs plus the
// 1 KiB pair of u slices that holds this tile's; only this tile's 512-byte
// slice is loaded into it (13 loads of 1 KiB and one of 512 bytes).
// Chunk j lives in slot j % RING.  The state wave reads it during chunk
// j - 1 and the output wave, two chunks behind, during chunk j + 2; the
// copy wave refills the slot with chunk j + RING during chunk
// j + RING - LEAD, and LEAD <= RING - 3 keeps that after both reads.  The
// copy wave issues chunk c + LEAD during chunk c and, before the barrier
// that ends chunk c, waits for chunk c + 2 (read by the state wave during
// chunk c + 1): its loads complete in issue order, so that wait leaves at
// most 14 * (LEAD - 2) loads outstanding.
constexpr int RING = 8;
constexpr int LEAD = 4;
// Hand-off slots from the state wave to the output wave: chunk c's hc and
// v_new are written during chunk c and read during chunk c + 2.
constexpr int HANDOFF = 4;
constexpr int SHARED_LOADS = REC_SHARED / 1024;  // 13
constexpr int LOADS_PER_CHUNK = SHARED_LOADS + 1;
constexpr int SLOT = REC_SHARED + 1024;
static_assert(SHARED_LOADS * 1024 == REC_SHARED, "shared part must be whole KiB");
static_assert(RING % HANDOFF == 0 && RING % 2 == 0, "slot indices follow the chunk index");
static_assert(LEAD >= 2 && LEAD <= RING - 3, "ring reuse order");
static_assert((LEAD - 1) * LOADS_PER_CHUNK <= 63, "vmcnt is a 6-bit count");
// The training recompute (no o) skips the record's qg: 10 loads a chunk.
constexpr int LOADS_NO_QG = LOADS_PER_CHUNK - (REC_KG - REC_QG) / 1024;
static_assert(REC_QG % 1024 == 0 && REC_KG - REC_QG == 4096, "qg is four whole loads");

// Hand-off from the state wave to the output wave, in slot c % HANDOFF:
// hc as the four 16x16x32 B operands (lane l's 16 bytes of operand j at
// 1024 * j + 16 * l) and v_new as the 16x16x16 B operand (8 bytes at 8 * l).
constexpr int HC_BYTES = 4 * 1024;
constexpr int VN_BYTES = 512;

// Copy wave: wait until the chunk followed by `n_after` issued chunks has
// landed (0 <= n_after <= LEAD - 2).
// NL: loads issued per chunk.
template <int N, int NL>
__device__ __forceinline__ void wait_chunk_ladder(int n_after) {
    if constexpr (N == 0) {
        wait_vmcnt<0>();
    } else {
        if (n_after >= N) {
            wait_vmcnt<N * NL>();
        } else {
            wait_chunk_ladder<N - 1, NL>(n_after);
        }
    }
}

template <int NL = LOADS_PER_CHUNK>
__device__ __forceinline__ void wait_chunk(int n_after) { wait_chunk_ladder<LEAD - 2, NL>(n_after); }

// One chunk's copy: 13 shared KiB, then this tile's 512-byte u slice (half
// a load: lanes 0-31) at its place in the slot's u pair, u_lds.  Buffer
// loads with the chunk offset in an SGPR and a fixed per-lane VGPR offset.
// NL == LOADS_NO_QG: without qg (its slot bytes are left as they were).
template <int NL = LOADS_PER_CHUNK>
__device__ __forceinline__ void issue_chunk(__amdgpu_buffer_rsrc_t rs, uint32_t chunk_off,
                                            lds_u8* slot, uint32_t u_off, uint32_t u_lds,
                                            uint32_t voff16) {
#pragma unroll
    for (int i = 0; i < SHARED_LOADS; ++i) {
        if (NL == LOADS_NO_QG && i >= REC_QG / 1024 && i < REC_KG / 1024) continue;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_u8*)(slot + i * 1024), 16, voff16,
                                                 chunk_off + i * 1024, 0, 0);
    }
    if (voff16 < 512)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_u8*)(slot + u_lds), 16, voff16,
                                                 chunk_off + u_off, 0, 0);
}

// The state wave's operands of one chunk.
struct StateOps {
    u32x4 w[4];
    u32x4 kg[4];
    // 2^G_last[16*kt + 4*q4 + i] for the two (kt, i) with 4*kt + i = 2*x and
    // 2*x + 1 (x = lane % 16); the 16 lanes of a row hold their row's 32.
    f32x2 dc;
    u32x2 u;
    u32x4 qg[4];  // split work-groups: the chunk's qg, for qg @ hc^T
};

// The prologue's read of chunk 0's operands (inside the loop the next
// chunk's operands are read piecewise, spread through the step).
// TPW > 1: a split work-group (below), whose slot holds the TPW u slices in
// tile order (ut: this wave's), and whose state wave also reads qg.
template <int TPW = 1>
__device__ __forceinline__ void read_state_ops_a(const uint8_t* slot, int lane, int vt,
                                                 StateOps& op, int ut = 0) {
    if constexpr (TPW > 1) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
            op.qg[j] = *reinterpret_cast<const u32x4*>(slot + REC_QG + j * 1024 + lane * 16);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j)
        op.w[j] = *reinterpret_cast<const u32x4*>(slot + REC_W + j * 1024 + lane * 16);
    op.u = *reinterpret_cast<const u32x2*>(slot + REC_SHARED + (TPW > 1 ? ut : vt & 1) * 512 + lane * 8);
#pragma unroll
    for (int j = 0; j < 4; ++j)
        op.kg[j] = *reinterpret_cast<const u32x4*>(slot + REC_KG + j * 1024 + lane * 16);
}

__device__ __forceinline__ void read_state_ops_b(const uint8_t* slot, int lane, StateOps& op) {
    op.dc = *reinterpret_cast<const f32x2*>(slot + decay_offset(lane));
}

// The record ring and the hand-off buffers of the work-group, referenced
// by name so that every address is a known LDS offset.  The direct loads
// take the ring as an LDS-space pointer, cast before any offset is applied.
__shared__ __attribute__((aligned(1024))) uint8_t ring[RING * SLOT];
__shared__ __attribute__((aligned(1024))) uint8_t hc_buf[HANDOFF][HC_BYTES];
__shared__ __attribute__((aligned(16))) uint8_t vn_buf[HANDOFF][VN_BYTES];

__device__ __forceinline__ lds_u8* ring_lds() { return (lds_u8*)ring; }

// Work-groups of TPW = 2 value tiles of one (sequence, head) (k2s_kernel
// below): one state wave per tile, one output wave for both, one copy wave.
// A ring slot holds the shared 13 KiB and the two u slices; the hand-off
// per tile and chunk is v_new and qg @ hc^T (fp32, 1 KiB), which the state
// wave forms itself, so the output wave reads neither hc nor qg.  (At four
// tiles the same structure ran slower than kda_k2w.hip's: B=1 T=8192 H=96
// forward 632 against 613 us.)
constexpr int QH_BYTES = 1024;
template <int TPW>
struct SplitLds {
    static constexpr int SLOT = REC_SHARED + TPW * 512;
    static constexpr int NL = SHARED_LOADS + TPW / 2;  // 1 KiB loads per chunk
    static_assert(TPW == 2, "two value tiles");
    static_assert((LEAD - 1) * NL <= 63, "vmcnt is a 6-bit count");
    static __device__ __forceinline__ uint8_t* ring();
    static __device__ __forceinline__ uint8_t* vn(int h, int ut);
    static __device__ __forceinline__ uint8_t* qh(int h, int ut);
};
__shared__ __attribute__((aligned(1024))) uint8_t ring_s2[RING * SplitLds<2>::SLOT];
__shared__ __attribute__((aligned(16))) uint8_t vn_s2[HANDOFF][2][VN_BYTES];
__shared__ __attribute__((aligned(16))) uint8_t qh_s2[HANDOFF][2][QH_BYTES];
template <> __device__ __forceinline__ uint8_t* SplitLds<2>::ring() { return ring_s2; }
template <> __device__ __forceinline__ uint8_t* SplitLds<2>::vn(int h, int ut) { return vn_s2[h][ut]; }
template <> __device__ __forceinline__ uint8_t* SplitLds<2>::qh(int h, int ut) { return qh_s2[h][ut]; }

// The state wave's barrier after a chunk that is followed by another: its
// last LDS accesses (the v_new hand-off, the next chunk's kg) need not be
// complete yet.  The hand-off a chunk writes is read two barriers later;
// every later chunk issues more than 15 LDS accesses before that barrier,
// and LDS accesses complete in order, so lgkmcnt(15) there covers it.
__device__ __forceinline__ void chunk_barrier_nodrain() {
    asm volatile("s_waitcnt lgkmcnt(15)\n\ts_barrier" ::: "memory");
    __builtin_amdgcn_s_waitcnt(WAITCNT_LGKM15);
}

// Constants of the chunk loop.
struct Ctx {
    __amdgpu_buffer_rsrc_t rs;  // copy: this sequence-head's records, NT * REC_BYTES bytes
    uint32_t voff16;            // copy: lane * 16
    uint32_t u_off;             // copy: REC_U + 512 * vt, this tile's u slice in the record
    uint32_t u_lds;             // copy: REC_SHARED + 512 * (vt % 2), its place in a ring slot
    uint16_t* obase;            // output: o[first token, hv, 16*vt + 4*((lane%16)/4)]
    int64_t orow_stride;        // output: elements between consecutive tokens of o
    uint16_t* trh;              // training: h of the first record, this tile, column 4*((lane%16)/4)
    uint16_t* trvn;             // training: v_new of the first record, likewise
    int rev;                    // backward: step c handles chunk NT - 1 - c
    float scale;
    int NT, T, lane, q4, vt;    // NT chunks over T tokens (this sequence's)
    int ut;                     // split work-groups: this state wave's tile among the TPW
};

// State wave, chunk c in ring slot S (a template argument, so every LDS
// offset is a compile-time constant).
//
// The step is software-pipelined across the chunk boundary: it starts with
// the state update of chunk c - 1,
//   S = S * 2^G_last + kg^T v_new      (kernels.py:281-294; S * 2^G_last
//                                       was formed during chunk c - 1),
// then forms chunk c's
//   hc = bf16(S),  v_new = bf16(u - w @ hc^T)   (kernels.py:261-266)
// with one accumulation chain that starts at u (the record holds -w), and
// hands hc and v_new to the output wave.  One wave issues at most one
// instruction per four cycles and stalls behind a matrix op the busy pipe
// cannot take, so the step is laid out by hand in small fenced groups that
// put VALU work (conversions, decay products, unpacking u) and LDS traffic
// (chunk c + 1's operands, the hand-off) behind each matrix op.
//
// op[S & 1] holds chunk c's operands.  op[(S + 1) & 1] holds chunk c - 1's
// until its kg has fed the update products, then receives chunk c + 1's.
// vn carries v_new from one step to the next.
//
// TPW > 1 (a split work-group): the slots and hand-offs of SplitLds<TPW>,
// and the state wave also forms qg @ hc^T, the first term of o, behind each
// w product (the output wave's order of products, so the same bits), and
// hands it off with v_new instead of hc.
template <int S, bool HAS_PREV, bool HAS_NEXT, int TPW = 1>
__device__ __forceinline__ void state_step(const Ctx& cx, f32x4 (&St)[8], StateOps (&op)[2],
                                           i16x4& vn) {
    constexpr bool QH = TPW > 1;
    const StateOps& cur = op[S & 1];
    StateOps& oth = op[(S + 1) & 1];
    const uint8_t* ns;
    if constexpr (QH) {
        ns = SplitLds<TPW>::ring() + ((S + 1) % RING) * SplitLds<TPW>::SLOT;
    } else {
        ns = ring + ((S + 1) % RING) * SLOT;
    }
    uint8_t* hbuf = hc_buf[S % HANDOFF] + cx.lane * 16;
    const int lane = cx.lane;

    auto update = [&](int kt) {  // tile kt of chunk c - 1's update
        if (HAS_PREV) {
            const u32x4 kg = oth.kg[kt >> 1];
            const u32x2 a = (kt & 1) ? u32x2{kg.z, kg.w} : u32x2{kg.x, kg.y};
            St[kt] = mfma_bf16_16x16x16(as_i16x4(a), vn, St[kt]);
        }
    };
    auto read_w = [&](int j) {
        if (HAS_NEXT) oth.w[j] = *reinterpret_cast<const u32x4*>(ns + REC_W + j * 1024 + lane * 16);
    };
    auto read_kg = [&](int j) {
        if (HAS_NEXT)
            oth.kg[j] = *reinterpret_cast<const u32x4*>(ns + REC_KG + j * 1024 + lane * 16);
    };
    auto read_dc = [&]() {
        if (HAS_NEXT) oth.dc = *reinterpret_cast<const f32x2*>(ns + decay_offset(lane));
    };
    auto read_qg = [&](int j) {
        if (QH && HAS_NEXT)
            oth.qg[j] = *reinterpret_cast<const u32x4*>(ns + REC_QG + j * 1024 + lane * 16);
    };
    const f32x4 zq = {0.f, 0.f, 0.f, 0.f};
    f32x4 qacc = zq;
    auto pack_hc = [&](int j) {  // bf16(S^T) of k-tiles 2j, 2j+1: a 16x16x32 B operand
        return u32x4{pack2(St[2 * j][0], St[2 * j][1]), pack2(St[2 * j][2], St[2 * j][3]),
                     pack2(St[2 * j + 1][0], St[2 * j + 1][1]),
                     pack2(St[2 * j + 1][2], St[2 * j + 1][3])};
    };
    auto decay = [&](auto jc) {
        constexpr int j = decltype(jc)::value;
        St[2 * j] = decay_tile<2 * j>(St[2 * j], cur.dc);
        St[2 * j + 1] = decay_tile<2 * j + 1>(St[2 * j + 1], cur.dc);
    };
#define KDA_FENCE() __builtin_amdgcn_sched_barrier(0)

    // Matrix pipe order: U0 U1 U2 U3 W0 U4 U5 W1 U6 U7 W2 W3 (Ukt: update
    // of tile kt, Wj: w product j).  Behind each, VALU work whose inputs
    // are done: hc_j needs U(2j), U(2j+1); decay_j follows hc_j.
    update(0);
    read_w(0);
    read_w(1);
    KDA_FENCE();
    update(1);
    read_w(2);
    read_w(3);
    read_qg(0);
    read_qg(1);
    // u as the fp32 accumulator the chain starts from
    const f32x4 u = {__builtin_bit_cast(float, cur.u.x << 16),
                     __builtin_bit_cast(float, cur.u.x & 0xffff0000u),
                     __builtin_bit_cast(float, cur.u.y << 16),
                     __builtin_bit_cast(float, cur.u.y & 0xffff0000u)};
    KDA_FENCE();
    update(2);
    const u32x4 hc0 = pack_hc(0);
    KDA_FENCE();
    update(3);
    decay(std::integral_constant<int, 0>{});
    KDA_FENCE();
    f32x4 va = mfma_bf16_16x16x32(as_bf16x8(cur.w[0]), as_bf16x8(hc0), u);
    if (QH) qacc = mfma_bf16_16x16x32(as_bf16x8(cur.qg[0]), as_bf16x8(hc0), zq);
    const u32x4 hc1 = pack_hc(1);
    if (HAS_NEXT)
        oth.u = *reinterpret_cast<const u32x2*>(ns + REC_SHARED + (QH ? cx.ut : cx.vt & 1) * 512 + lane * 8);
    read_dc();
    KDA_FENCE();
    update(4);
    decay(std::integral_constant<int, 1>{});
    KDA_FENCE();
    update(5);
    KDA_FENCE();
    va = mfma_bf16_16x16x32(as_bf16x8(cur.w[1]), as_bf16x8(hc1), va);
    if (QH) {
        qacc = mfma_bf16_16x16x32(as_bf16x8(cur.qg[1]), as_bf16x8(hc1), qacc);
        read_qg(2);
        read_qg(3);
    } else {
        *reinterpret_cast<u32x4*>(hbuf + 0 * 1024) = hc0;
        *reinterpret_cast<u32x4*>(hbuf + 1 * 1024) = hc1;
    }
    KDA_FENCE();
    update(6);
    const u32x4 hc2 = pack_hc(2);
    KDA_FENCE();
    update(7);
    decay(std::integral_constant<int, 2>{});
    KDA_FENCE();
    va = mfma_bf16_16x16x32(as_bf16x8(cur.w[2]), as_bf16x8(hc2), va);
    if (QH) qacc = mfma_bf16_16x16x32(as_bf16x8(cur.qg[2]), as_bf16x8(hc2), qacc);
    const u32x4 hc3 = pack_hc(3);
    KDA_FENCE();
    va = mfma_bf16_16x16x32(as_bf16x8(cur.w[3]), as_bf16x8(hc3), va);
    if (QH) qacc = mfma_bf16_16x16x32(as_bf16x8(cur.qg[3]), as_bf16x8(hc3), qacc);
    decay(std::integral_constant<int, 3>{});
    if (!QH) {
        *reinterpret_cast<u32x4*>(hbuf + 2 * 1024) = hc2;
        *reinterpret_cast<u32x4*>(hbuf + 3 * 1024) = hc3;
    }
    read_kg(0);
    read_kg(1);
    read_kg(2);
    read_kg(3);
    KDA_FENCE();

    const u32x2 vnb = {pack2(va[0], va[1]), pack2(va[2], va[3])};
    if constexpr (QH) {
        // (with the reads above, 16 LDS accesses a step: the barrier rule holds)
        *reinterpret_cast<u32x2*>(SplitLds<TPW>::vn(S % HANDOFF, cx.ut) + lane * 8) = vnb;
        *reinterpret_cast<f32x4*>(SplitLds<TPW>::qh(S % HANDOFF, cx.ut) + lane * 16) = qacc;
    } else {
        *reinterpret_cast<u32x2*>(vn_buf[S % HANDOFF] + lane * 8) = vnb;
    }
    vn = as_i16x4(vnb);
    if (HAS_NEXT) {
        chunk_barrier_nodrain();
    } else {
        chunk_barrier();
    }
    KDA_FENCE();
    if (!HAS_NEXT) {
        // the last chunk's update
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const u32x2 k0 = {cur.kg[j].x, cur.kg[j].y};
            const u32x2 k1 = {cur.kg[j].z, cur.kg[j].w};
            St[2 * j] = mfma_bf16_16x16x16(as_i16x4(k0), vn, St[2 * j]);
            St[2 * j + 1] = mfma_bf16_16x16x16(as_i16x4(k1), vn, St[2 * j + 1]);
        }
    }
#undef KDA_FENCE
}

// Output wave, chunk c (slot S) after the barrier that ends chunk c + 1:
// o = scale * qg @ hc^T + Aqk @ v_new (kernels.py:268-279).
// TRAIN: instead of o, store the chunk's hc = bf16(S) as h = hc^T and
// v_new into the backward's training buffers (blocked by value tile, so a
// k-tile of this work-group is 512 contiguous bytes), each 16x16 tile
// quad-transposed to one 8-byte row piece per lane.
// Two store waves share that work (PART 0: k-tiles 0-3, PART 1: k-tiles
// 4-7 and v_new); a single wave would fall behind the state wave.
// WITH_O (a training forward that saves its state): o as well, after the
// training stores.
template <int S, bool TRAIN, int PART, bool WITH_O = !TRAIN>
__device__ __forceinline__ void output_step(const Ctx& cx, int c) {
    chunk_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (TRAIN) {
        const int j4 = cx.lane & 3;
        const int cs = cx.rev ? cx.NT - 1 - c : c;  // the chunk of step c
        uint16_t* hrec = cx.trh + (int64_t)cs * TR_H_ELEMS;
#pragma unroll
        for (int j = 2 * PART; j < 2 * PART + 2; ++j) {
            const u32x4 hc = *reinterpret_cast<const u32x4*>(hc_buf[S % HANDOFF] + j * 1024 + cx.lane * 16);
            const u32x2 t0 = quad_transpose(hc.x, hc.y, j4);
            const u32x2 t1 = quad_transpose(hc.z, hc.w, j4);
            const int k0 = 32 * j + 4 * cx.q4 + j4;  // row of k-tile 2j
            __builtin_nontemporal_store(t0, reinterpret_cast<u32x2*>(hrec + k0 * 16));
            __builtin_nontemporal_store(t1, reinterpret_cast<u32x2*>(hrec + (k0 + 16) * 16));
        }
        if (PART == 1) {
            const u32x2 vn = *reinterpret_cast<const u32x2*>(vn_buf[S % HANDOFF] + cx.lane * 8);
            const u32x2 vt = quad_transpose(vn.x, vn.y, j4);
            __builtin_nontemporal_store(
                vt, reinterpret_cast<u32x2*>(cx.trvn + (int64_t)cs * TR_VN_ELEMS + (4 * cx.q4 + j4) * 16));
        }
        if constexpr (!WITH_O) return;
    }
    const uint8_t* slot = ring + S * SLOT;
    u32x4 hc[4], qg[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        hc[j] = *reinterpret_cast<const u32x4*>(hc_buf[S % HANDOFF] + j * 1024 + cx.lane * 16);
        qg[j] = *reinterpret_cast<const u32x4*>(slot + REC_QG + j * 1024 + cx.lane * 16);
    }
    const u32x2 vn = *reinterpret_cast<const u32x2*>(vn_buf[S % HANDOFF] + cx.lane * 8);
    // Aqk is read 16 bytes at a time (this lane's 8 and its neighbour's):
    // the compiler puts a vmcnt(0) before an 8-byte LDS read of the ring
    // here, which would wait for this wave's own stores.
    const u32x4 aq2 = *reinterpret_cast<const u32x4*>(slot + REC_AQK + (cx.lane >> 1) * 16);
    const u32x2 aqk = (cx.lane & 1) ? u32x2{aq2.z, aq2.w} : u32x2{aq2.x, aq2.y};
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    f32x4 oacc = mfma_bf16_16x16x32(as_bf16x8(qg[0]), as_bf16x8(hc[0]), zero);
#pragma unroll
    for (int j = 1; j < 4; ++j)
        oacc = mfma_bf16_16x16x32(as_bf16x8(qg[j]), as_bf16x8(hc[j]), oacc);
    oacc = oacc * cx.scale;
    oacc = mfma_bf16_16x16x16(as_i16x4(aqk), as_i16x4(vn), oacc);
    // Lane (x, q4) holds o rows 4*q4 .. +3 of column x; after the quad
    // transpose it holds row 4*q4 + x%4, columns 4*(x/4) .. +3.
    const u32x2 ot = quad_transpose(pack2(oacc[0], oacc[1]), pack2(oacc[2], oacc[3]), cx.lane & 3);
    const int t = c * BT + 4 * cx.q4 + (cx.lane & 3);
    // o is written once and never read back here: a non-temporal store.
    if (t < cx.T)
        __builtin_nontemporal_store(ot, reinterpret_cast<u32x2*>(cx.obase + (int64_t)t * cx.orow_stride));
}

// Record offset of step c's chunk (in reverse order for the backward).
__device__ __forceinline__ uint32_t step_rec(const Ctx& cx, int c) {
    return (uint32_t)(cx.rev ? cx.NT - 1 - c : c) * REC_BYTES;
}

// Copy wave, chunk c (slot S); NL loads a chunk.
template <int S, int NL>
__device__ __forceinline__ void copy_step(const Ctx& cx, int c) {
    if (c + LEAD < cx.NT)
        issue_chunk<NL>(cx.rs, step_rec(cx, c + LEAD),
                        ring_lds() + ((S + LEAD) % RING) * SLOT, cx.u_off, cx.u_lds, cx.voff16);
    // chunk c + 2 is read by the state wave after this barrier
    if (c + 2 < cx.NT) wait_chunk<NL>(min(LEAD - 2, cx.NT - 3 - c));
    copy_barrier();
}

// One pass over the ring: chunks c .. c + RING - 1 (those below NT), each
// with its slot as a compile-time constant.
// N chunks from slot S on, each followed by another (so with a next
// chunk to prefetch) and preceded by one.
template <int S, int N, int TPW = 1>
__device__ __forceinline__ void state_round_full(const Ctx& cx, f32x4 (&St)[8],
                                                 StateOps (&op)[2], i16x4& vn) {
    state_step<S, true, true, TPW>(cx, St, op, vn);
    if constexpr (N > 1) state_round_full<(S + 1) % RING, N - 1, TPW>(cx, St, op, vn);
}

// The remaining chunks c .. NT - 1 (at most N of them) from slot S on.
template <int S, int N, int TPW = 1>
__device__ __forceinline__ void state_round_tail(const Ctx& cx, int c, f32x4 (&St)[8],
                                                 StateOps (&op)[2], i16x4& vn) {
    if (c >= cx.NT) return;
    if (c + 1 < cx.NT) {
        state_step<S, true, true, TPW>(cx, St, op, vn);
    } else {
        state_step<S, true, false, TPW>(cx, St, op, vn);
    }
    if constexpr (N > 1) state_round_tail<(S + 1) % RING, N - 1, TPW>(cx, c + 1, St, op, vn);
}

template <int S, bool TRAIN, int PART, bool WITH_O>
__device__ __forceinline__ void output_round(const Ctx& cx, int c) {
    output_step<S, TRAIN, PART, WITH_O>(cx, c);
    if constexpr (S + 1 < RING) {
        if (c + 1 < cx.NT) output_round<S + 1, TRAIN, PART, WITH_O>(cx, c + 1);
    }
}

template <int S, int NL>
__device__ __forceinline__ void copy_round(const Ctx& cx, int c) {
    copy_step<S, NL>(cx, c);
    if constexpr (S + 1 < RING) {
        if (c + 1 < cx.NT) copy_round<S + 1, NL>(cx, c + 1);
    }
}

template <int NL = LOADS_PER_CHUNK>
__device__ __forceinline__ void copy_wave(const Params& p, Ctx& cx, const SeqSpan& sp) {
    const int NT = cx.NT;
    uint8_t* recs = cx.rev ? p.ws_bwd + sp.srec0 * REC_BYTES : p.ws + sp.rec0 * REC_BYTES;
    cx.rs = __builtin_amdgcn_make_buffer_rsrc(recs, (short)0, NT * REC_BYTES, BUF_DWORD3);
    cx.voff16 = cx.lane * 16;
    cx.u_off = REC_U + 512 * cx.vt;
    cx.u_lds = REC_SHARED + 512 * (cx.vt & 1);
#pragma unroll
    for (int d = 0; d < LEAD; ++d)
        if (d < NT)
            issue_chunk<NL>(cx.rs, step_rec(cx, d), ring_lds() + d * SLOT, cx.u_off, cx.u_lds,
                            cx.voff16);
    // chunks 0 and 1 (those that exist) before the first barrier
    wait_chunk<NL>(NT >= 2 ? min(LEAD, NT) - 2 : 0);
    copy_barrier();
    for (int c = 0; c < NT; c += RING) copy_round<0, NL>(cx, c);
    copy_barrier();  // the output wave's last chunk
}

template <bool TRAIN, int PART, bool WITH_O = !TRAIN>
__device__ __forceinline__ void output_wave(const Params& p, Ctx& cx, const SeqSpan& sp, int hv) {
    const int x = cx.lane & 15;
    const int col = 16 * cx.vt + 4 * (x >> 2);
    if constexpr (TRAIN) {
        // forward recompute: h and v_new; backward: dh' and dv_new
        uint16_t* bh = cx.rev ? p.tr_dh : p.tr_h;
        uint16_t* bv = cx.rev ? p.tr_dvn : p.tr_vn;
        cx.trh = bh + sp.srec0 * TR_H_ELEMS + cx.vt * TR_H_TILE + 4 * (x >> 2);
        cx.trvn = bv + sp.srec0 * TR_VN_ELEMS + cx.vt * TR_VN_TILE + 4 * (x >> 2);
    }
    if constexpr (WITH_O) {
        cx.obase = p.o + (sp.tok0 * p.HV + hv) * DK + col;
        cx.orow_stride = (int64_t)p.HV * DK;
    }
    chunk_barrier();
    chunk_barrier();
    for (int c = 0; c < cx.NT; c += RING) output_round<0, TRAIN, PART, WITH_O>(cx, c);
}

// ---------------------------------------------------------------------------
// Backward: the reverse recurrence of the state gradient dh (K x 16 of this
// value tile, the layout of S^T above).  Step c handles chunk NT - 1 - c:
//   dv_new = Aqk^T dO + kg dh'
//   dh     = 2^G_last * dh' + [scale qg | -w]^T [dO ; dv_new]
// with dh' the gradient of the state after the chunk.  The record (stage
// 1's backward record) holds every operand in register order: kg where the
// forward keeps w, the eight [scale qg | -w]^T tiles over qg and kg, Aqk^T
// over Aqk, and this tile's dO where the forward keeps u.  dh' and dv_new go
// to the output wave through the hand-off, as hc and v_new do forward.
// ---------------------------------------------------------------------------

struct BwdStateOps {
    u32x4 kg[4];
    u32x4 upd[8];
    u32x2 aqkT;
    u32x2 dop;
    f32x2 dc;
};

__device__ __forceinline__ void read_bwd_ops(const uint8_t* slot, int lane, int vt, BwdStateOps& op) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
        op.kg[j] = *reinterpret_cast<const u32x4*>(slot + BREC_KG + j * 1024 + lane * 16);
#pragma unroll
    for (int kt = 0; kt < 8; ++kt)
        op.upd[kt] = *reinterpret_cast<const u32x4*>(slot + BREC_UPD + kt * 1024 + lane * 16);
    op.aqkT = *reinterpret_cast<const u32x2*>(slot + BREC_AQKT + lane * 8);
    op.dop = *reinterpret_cast<const u32x2*>(slot + REC_SHARED + (vt & 1) * 512 + lane * 8);
    op.dc = *reinterpret_cast<const f32x2*>(slot + decay_offset(lane));
}

// dh[kt] = 2^G_last * dh[kt] + upd[kt] @ [dO ; dv_new] for one step's ops.
template <int KT>
__device__ __forceinline__ void bwd_update(f32x4 (&D)[8], const BwdStateOps& o, const u32x4& bop) {
    D[KT] = decay_tile<KT>(D[KT], o.dc);
    D[KT] = mfma_bf16_16x16x32(as_bf16x8(o.upd[KT]), as_bf16x8(bop), D[KT]);
}

__device__ __forceinline__ u32x4 pack_tiles(const f32x4& a, const f32x4& b) {
    return u32x4{pack2(a[0], a[1]), pack2(a[2], a[3]), pack2(b[0], b[1]), pack2(b[2], b[3])};
}

// Step c in slot S, software-pipelined as the forward's state_step: it
// starts with step c - 1's update, tile by tile, and runs this step's
// kg @ dh' chain as soon as the tiles it needs are updated.  op[(S+1) & 1]
// holds step c - 1's operands until its update is done, then receives step
// c + 1's; bop carries [dO ; dv_new] of step c - 1 in, of step c out.
template <int S, bool HAS_PREV, bool HAS_NEXT>
__device__ __forceinline__ void bwd_state_step(const Ctx& cx, f32x4 (&D)[8], BwdStateOps (&op)[2],
                                               u32x4& bop) {
    const BwdStateOps& cur = op[S & 1];
    BwdStateOps& oth = op[(S + 1) & 1];
    const uint8_t* ns = ring + ((S + 1) % RING) * SLOT;
    uint8_t* hbuf = hc_buf[S % HANDOFF] + cx.lane * 16;
#define KDA_FENCE() __builtin_amdgcn_sched_barrier(0)
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    // Aqk^T dO in the 16x16x32 shape of the chain it starts
    f32x4 dvn = mfma_bf16_16x16x16_in_x32(cur.aqkT, cur.dop, zero);
    if (HAS_PREV) {
        bwd_update<0>(D, oth, bop);
        bwd_update<1>(D, oth, bop);
    }
    KDA_FENCE();
    const u32x4 hb0 = pack_tiles(D[0], D[1]);
    dvn = mfma_bf16_16x16x32(as_bf16x8(cur.kg[0]), as_bf16x8(hb0), dvn);
    if (HAS_PREV) {
        bwd_update<2>(D, oth, bop);
        bwd_update<3>(D, oth, bop);
    }
    *reinterpret_cast<u32x4*>(hbuf + 0 * 1024) = hb0;
    KDA_FENCE();
    const u32x4 hb1 = pack_tiles(D[2], D[3]);
    dvn = mfma_bf16_16x16x32(as_bf16x8(cur.kg[1]), as_bf16x8(hb1), dvn);
    if (HAS_PREV) {
        bwd_update<4>(D, oth, bop);
        bwd_update<5>(D, oth, bop);
    }
    *reinterpret_cast<u32x4*>(hbuf + 1 * 1024) = hb1;
    KDA_FENCE();
    const u32x4 hb2 = pack_tiles(D[4], D[5]);
    dvn = mfma_bf16_16x16x32(as_bf16x8(cur.kg[2]), as_bf16x8(hb2), dvn);
    if (HAS_PREV) {
        bwd_update<6>(D, oth, bop);
        bwd_update<7>(D, oth, bop);
    }
    *reinterpret_cast<u32x4*>(hbuf + 2 * 1024) = hb2;
    KDA_FENCE();
    const u32x4 hb3 = pack_tiles(D[6], D[7]);
    dvn = mfma_bf16_16x16x32(as_bf16x8(cur.kg[3]), as_bf16x8(hb3), dvn);
    *reinterpret_cast<u32x4*>(hbuf + 3 * 1024) = hb3;
    if (HAS_NEXT) read_bwd_ops(ns, cx.lane, cx.vt, oth);
    KDA_FENCE();
    const u32x2 dvb = {pack2(dvn[0], dvn[1]), pack2(dvn[2], dvn[3])};
    *reinterpret_cast<u32x2*>(vn_buf[S % HANDOFF] + cx.lane * 8) = dvb;
    bop = u32x4{cur.dop.x, cur.dop.y, dvb.x, dvb.y};
    if (HAS_NEXT) {
        chunk_barrier_nodrain();
    } else {
        chunk_barrier();
    }
    KDA_FENCE();
    if (!HAS_NEXT) {
        // the last step's update: dh becomes the initial state's gradient
        bwd_update<0>(D, cur, bop);
        bwd_update<1>(D, cur, bop);
        bwd_update<2>(D, cur, bop);
        bwd_update<3>(D, cur, bop);
        bwd_update<4>(D, cur, bop);
        bwd_update<5>(D, cur, bop);
        bwd_update<6>(D, cur, bop);
        bwd_update<7>(D, cur, bop);
    }
#undef KDA_FENCE
}

template <int S, int N>
__device__ __forceinline__ void bwd_round_full(const Ctx& cx, f32x4 (&D)[8], BwdStateOps (&op)[2],
                                               u32x4& bop) {
    bwd_state_step<S, true, true>(cx, D, op, bop);
    if constexpr (N > 1) bwd_round_full<(S + 1) % RING, N - 1>(cx, D, op, bop);
}

template <int S, int N>
__device__ __forceinline__ void bwd_round_tail(const Ctx& cx, int c, f32x4 (&D)[8],
                                               BwdStateOps (&op)[2], u32x4& bop) {
    if (c >= cx.NT) return;
    if (c + 1 < cx.NT) {
        bwd_state_step<S, true, true>(cx, D, op, bop);
    } else {
        bwd_state_step<S, true, false>(cx, D, op, bop);
    }
    if constexpr (N > 1) bwd_round_tail<(S + 1) % RING, N - 1>(cx, c + 1, D, op, bop);
}

__device__ __forceinline__ void bwd_state_wave(const Params& p, const Ctx& cx, int bh) {
    const int lane = cx.lane, q4 = cx.q4, vt = cx.vt;
    const int v = 16 * vt + (lane & 15);
    const int64_t sbase = (int64_t)bh * DK * DK;
    f32x4 D[8];
    load_state_from(p.dht ? p.dht + sbase : nullptr, p.h0_v_first != 0, v, q4, D);
    chunk_barrier();  // steps 0 and 1 are in the ring
    BwdStateOps op[2];
    read_bwd_ops(ring, lane, vt, op[0]);
    __builtin_amdgcn_s_waitcnt(WAITCNT_LGKM0);
    u32x4 bop;
    if (cx.NT > 1) {
        bwd_state_step<0, false, true>(cx, D, op, bop);
    } else {
        bwd_state_step<0, false, false>(cx, D, op, bop);
    }
    int c = 1;
    for (; c + RING < cx.NT; c += RING) bwd_round_full<1, RING>(cx, D, op, bop);
    bwd_round_tail<1 % RING, RING>(cx, c, D, op, bop);
    chunk_barrier();  // the output wave's last step
    store_state_to(p.dh0 ? p.dh0 + sbase : nullptr, p.h0_v_first != 0, v, q4, D);
}

template <int TPW = 1>
__device__ __forceinline__ void state_wave(const Params& p, const Ctx& cx, int bh) {
    const int lane = cx.lane, q4 = cx.q4, vt = cx.vt;
    const int v = 16 * vt + (lane & 15);
    const int64_t sbase = (int64_t)bh * DK * DK;
    f32x4 St[8];
    load_state(p, sbase, v, q4, St);
    chunk_barrier();  // chunks 0 and 1 are in the ring
    StateOps op[2];
    const uint8_t* slot0;
    if constexpr (TPW > 1) {
        slot0 = SplitLds<TPW>::ring();
    } else {
        slot0 = ring;
    }
    read_state_ops_a<TPW>(slot0, lane, vt, op[0], cx.ut);
    read_state_ops_b(slot0, lane, op[0]);
    __builtin_amdgcn_s_waitcnt(WAITCNT_LGKM0);
    i16x4 vn;
    if (cx.NT > 1) {
        state_step<0, false, true, TPW>(cx, St, op, vn);
    } else {
        state_step<0, false, false, TPW>(cx, St, op, vn);
    }
    int c = 1;
    for (; c + RING < cx.NT; c += RING) state_round_full<1, RING, TPW>(cx, St, op, vn);
    state_round_tail<1 % RING, RING, TPW>(cx, c, St, op, vn);
    chunk_barrier();  // the output wave's last chunk
    store_state(p, sbase, v, q4, St);
}

// ---------------------------------------------------------------------------
// Several sequences per work-group (forward).  With more (sequence, head,
// value tile) triples than CUs, one work-group per triple would run in
// rounds, each paying its own ring fill and drain.  Instead a work-group
// takes a (group of sequences, value head, value tile) and runs the chunks
// of its sequences as one stream of steps through the same ring: step j is
// chunk c of sequence n in walk order.  At the first chunk of a sequence
// the state wave finishes the previous sequence (its last update, its
// final state stored), loads the new initial state (one load latency per
// sequence) and runs the step without the previous update.  The copy and
// output waves only follow the walk to address records and o rows.  The
// state wave keeps no load in flight across steps: a pending load would
// make the compiler's waits in later steps cover the final-state stores
// too.
// ---------------------------------------------------------------------------

// Position in the walk over the non-empty sequences [.., n_end) of a group.
struct SeqWalk {
    int n, n_end;  // current sequence (n_end once past the last)
    int c;         // chunk within it
    SeqSpan sp;    // its span (value head hv)
};

// Moves to the first non-empty sequence at or after n.
__device__ __forceinline__ void walk_seek(const Params& p, int hv, SeqWalk& w, int n) {
    for (; n < w.n_end; ++n) {
        w.sp = seq_span(p, n * p.HV + hv);
        if (w.sp.nt > 0) break;
    }
    w.n = n;
    w.c = 0;
}

__device__ __forceinline__ void walk_init(const Params& p, int hv, int n0, int n1, SeqWalk& w) {
    w.n_end = n1;
    walk_seek(p, hv, w, n0);
}

__device__ __forceinline__ void walk_advance(const Params& p, int hv, SeqWalk& w) {
    if (++w.c == w.sp.nt) walk_seek(p, hv, w, w.n + 1);
}


struct MsCtx {
    int hv, n0, n1, J;  // value head, sequences [n0, n1), steps
};

// The state wave's step j in slot S.  At a sequence's first chunk a short
// boundary block comes first (rare, kept off the hot path): the previous
// sequence's last update (chunk j - 1) and its final state, then the new
// initial state.  v_new is then zeroed, so the step's own update of chunk
// j - 1 adds exact zeros, and every step runs the one pipelined body.
template <int S, bool HAS_NEXT>
__device__ __forceinline__ void state_step_ms(const Params& p, const Ctx& cx, const MsCtx& m,
                                              f32x4 (&St)[8], StateOps (&op)[2], i16x4& vn,
                                              SeqWalk& w, int& last_n) {
    if (__builtin_expect(w.c == 0, 0)) {
        const int v = 16 * cx.vt + (cx.lane & 15);
        const StateOps& prev = op[(S + 1) & 1];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const u32x2 k0 = {prev.kg[j].x, prev.kg[j].y};
            const u32x2 k1 = {prev.kg[j].z, prev.kg[j].w};
            St[2 * j] = mfma_bf16_16x16x16(as_i16x4(k0), vn, St[2 * j]);
            St[2 * j + 1] = mfma_bf16_16x16x16(as_i16x4(k1), vn, St[2 * j + 1]);
        }
        store_state(p, ((int64_t)last_n * p.HV + m.hv) * DK * DK, v, cx.q4, St);
        load_state(p, ((int64_t)w.n * p.HV + m.hv) * DK * DK, v, cx.q4, St);
        vn = i16x4{0, 0, 0, 0};
    }
    state_step<S, true, HAS_NEXT>(cx, St, op, vn);
    last_n = w.n;
    walk_advance(p, m.hv, w);
}

// A round with no sequence boundary: the plain pipelined steps (the same
// code as one sequence per work-group, so the hot loop stays compact).
template <int S, int N>
__device__ __forceinline__ void state_round_plain(const Ctx& cx, f32x4 (&St)[8], StateOps (&op)[2],
                                                  i16x4& vn) {
    state_step<S, true, true>(cx, St, op, vn);
    if constexpr (N > 1) state_round_plain<(S + 1) % RING, N - 1>(cx, St, op, vn);
}

template <int S, int N>
__device__ __forceinline__ void state_round_full_ms(const Params& p, const Ctx& cx, const MsCtx& m,
                                                    f32x4 (&St)[8], StateOps (&op)[2], i16x4& vn,
                                                    SeqWalk& w, int& last_n) {
    state_step_ms<S, true>(p, cx, m, St, op, vn, w, last_n);
    if constexpr (N > 1)
        state_round_full_ms<(S + 1) % RING, N - 1>(p, cx, m, St, op, vn, w, last_n);
}

template <int S, int N>
__device__ __forceinline__ void state_round_tail_ms(const Params& p, const Ctx& cx, const MsCtx& m,
                                                    int j, f32x4 (&St)[8], StateOps (&op)[2],
                                                    i16x4& vn, SeqWalk& w, int& last_n) {
    if (j >= m.J) return;
    if (j + 1 < m.J) {
        state_step_ms<S, true>(p, cx, m, St, op, vn, w, last_n);
    } else {
        state_step_ms<S, false>(p, cx, m, St, op, vn, w, last_n);
    }
    if constexpr (N > 1)
        state_round_tail_ms<(S + 1) % RING, N - 1>(p, cx, m, j + 1, St, op, vn, w, last_n);
}

__device__ __forceinline__ void state_wave_ms(const Params& p, const Ctx& cx, const MsCtx& m) {
    const int lane = cx.lane, q4 = cx.q4;
    const int v = 16 * cx.vt + (lane & 15);
    // an empty sequence's final state is its initial state
    for (int n = m.n0; n < m.n1; ++n) {
        if (seq_span(p, n * p.HV + m.hv).nt == 0) {
            f32x4 E[8];
            const int64_t sb = ((int64_t)n * p.HV + m.hv) * DK * DK;
            load_state(p, sb, v, q4, E);
            store_state(p, sb, v, q4, E);
        }
    }
    if (m.J == 0) return;
    SeqWalk w;
    walk_init(p, m.hv, m.n0, m.n1, w);
    f32x4 St[8];
    load_state(p, ((int64_t)w.n * p.HV + m.hv) * DK * DK, v, q4, St);
    chunk_barrier();  // chunks 0 and 1 are in the ring
    StateOps op[2];
    read_state_ops_a(ring, lane, cx.vt, op[0]);
    read_state_ops_b(ring, lane, op[0]);
    __builtin_amdgcn_s_waitcnt(WAITCNT_LGKM0);
    i16x4 vn;
    if (m.J > 1) {
        state_step<0, false, true>(cx, St, op, vn);
    } else {
        state_step<0, false, false>(cx, St, op, vn);
    }
    int last_n = w.n;
    walk_advance(p, m.hv, w);
    // Rounds of RING steps from step 1 on.  Rounds without a boundary run
    // in an inner loop of their own, so that what the boundary rounds keep
    // live is not live there.
    int j = 1;
    while (j + RING < m.J) {
        while (j + RING < m.J && w.c != 0 && w.sp.nt - w.c >= RING) {
            state_round_plain<1, RING>(cx, St, op, vn);
            last_n = w.n;
            w.c += RING;
            if (w.c == w.sp.nt) walk_seek(p, m.hv, w, w.n + 1);
            j += RING;
        }
        if (j + RING < m.J) {
            state_round_full_ms<1, RING>(p, cx, m, St, op, vn, w, last_n);
            j += RING;
        }
    }
    state_round_tail_ms<1 % RING, RING>(p, cx, m, j, St, op, vn, w, last_n);
    chunk_barrier();  // the output wave's last chunk
    store_state(p, ((int64_t)last_n * p.HV + m.hv) * DK * DK, v, q4, St);
}

template <int S>
__device__ __forceinline__ void output_round_ms(const Params& p, Ctx& cx, const MsCtx& m, int j,
                                                SeqWalk& w) {
    cx.obase = p.o + (w.sp.tok0 * p.HV + m.hv) * DK + 16 * cx.vt + 4 * ((cx.lane & 15) >> 2);
    cx.T = w.sp.len;
    output_step<S, false, 0>(cx, w.c);
    walk_advance(p, m.hv, w);
    if constexpr (S + 1 < RING) {
        if (j + 1 < m.J) output_round_ms<S + 1>(p, cx, m, j + 1, w);
    }
}

__device__ __forceinline__ void output_wave_ms(const Params& p, Ctx& cx, const MsCtx& m) {
    if (m.J == 0) return;
    SeqWalk w;
    walk_init(p, m.hv, m.n0, m.n1, w);
    cx.orow_stride = (int64_t)p.HV * DK;
    chunk_barrier();
    chunk_barrier();
    for (int j = 0; j < m.J; j += RING) output_round_ms<0>(p, cx, m, j, w);
}

// Issues the record of the walk's current step into `slot`.
__device__ __forceinline__ void issue_ms(const Params& p, const Ctx& cx, const SeqWalk& w,
                                         lds_u8* slot) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        p.ws + w.sp.rec0 * REC_BYTES, (short)0, w.sp.nt * REC_BYTES, BUF_DWORD3);
    issue_chunk(rs, (uint32_t)w.c * REC_BYTES, slot, cx.u_off, cx.u_lds, cx.voff16);
}

template <int S>
__device__ __forceinline__ void copy_round_ms(const Params& p, const Ctx& cx, const MsCtx& m,
                                              int j, SeqWalk& w) {
    if (j + LEAD < m.J) {
        issue_ms(p, cx, w, ring_lds() + ((S + LEAD) % RING) * SLOT);
        walk_advance(p, m.hv, w);
    }
    if (j + 2 < m.J) wait_chunk(min(LEAD - 2, m.J - 3 - j));
    copy_barrier();
    if constexpr (S + 1 < RING) {
        if (j + 1 < m.J) copy_round_ms<S + 1>(p, cx, m, j + 1, w);
    }
}

__device__ __forceinline__ void copy_wave_ms(const Params& p, Ctx& cx, const MsCtx& m) {
    if (m.J == 0) return;
    SeqWalk w;
    walk_init(p, m.hv, m.n0, m.n1, w);
    cx.voff16 = cx.lane * 16;
    cx.u_off = REC_U + 512 * cx.vt;
    cx.u_lds = REC_SHARED + 512 * (cx.vt & 1);
#pragma unroll
    for (int d = 0; d < LEAD; ++d) {
        if (d < m.J) {
            issue_ms(p, cx, w, ring_lds() + d * SLOT);
            walk_advance(p, m.hv, w);
        }
    }
    wait_chunk(m.J >= 2 ? min(LEAD, m.J) - 2 : 0);
    copy_barrier();
    for (int j = 0; j < m.J; j += RING) copy_round_ms<0>(p, cx, m, j, w);
    copy_barrier();  // the output wave's last chunk
}

// ---------------------------------------------------------------------------
// Split work-groups (k2s_kernel): TPW = 2 value tiles of one (sequence,
// head), one state wave per tile (state_step with its qg @ hc^T), one output
// wave for both tiles, one copy wave streaming each record once (the shared
// 13 KiB and the two u slices).  Where one-tile work-groups would outnumber
// the CUs by up to twice, this shares the record stream between the tiles
// as kda_k2w.hip does, while each tile's recurrence keeps a wave of its own
// with little but the chain on it.  Same ring, lead, hand-off depth and
// barrier per chunk as the one-tile kernel; o bit for bit that kernel's.
// ---------------------------------------------------------------------------

// Copy wave: one chunk's 13 shared KiB, then the TPW u slices (TPW / 2
// loads of 1 KiB), at their places in the slot.
template <int TPW>
__device__ __forceinline__ void issue_chunk_split(__amdgpu_buffer_rsrc_t rs, uint32_t chunk_off,
                                                  lds_u8* slot, uint32_t u_off, uint32_t voff16) {
#pragma unroll
    for (int i = 0; i < SHARED_LOADS; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_u8*)(slot + i * 1024), 16, voff16,
                                                 chunk_off + i * 1024, 0, 0);
#pragma unroll
    for (int i = 0; i < TPW / 2; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_u8*)(slot + REC_SHARED + i * 1024), 16,
                                                 voff16, chunk_off + u_off + i * 1024, 0, 0);
}

template <int S, int TPW>
__device__ __forceinline__ void copy_round_split(const Ctx& cx, int c) {
    using L = SplitLds<TPW>;
    if (c + LEAD < cx.NT)
        issue_chunk_split<TPW>(cx.rs, (uint32_t)(c + LEAD) * REC_BYTES,
                               (lds_u8*)L::ring() + ((S + LEAD) % RING) * L::SLOT, cx.u_off, cx.voff16);
    // chunk c + 2 is read by the state waves after this barrier
    if (c + 2 < cx.NT) wait_chunk<L::NL>(min(LEAD - 2, cx.NT - 3 - c));
    copy_barrier();
    if constexpr (S + 1 < RING) {
        if (c + 1 < cx.NT) copy_round_split<S + 1, TPW>(cx, c + 1);
    }
}

template <int TPW>
__device__ __forceinline__ void copy_wave_split(const Params& p, Ctx& cx, const SeqSpan& sp, int slice) {
    using L = SplitLds<TPW>;
    const int NT = cx.NT;
    cx.rs = __builtin_amdgcn_make_buffer_rsrc(p.ws + sp.rec0 * REC_BYTES, (short)0, NT * REC_BYTES,
                                              BUF_DWORD3);
    cx.voff16 = cx.lane * 16;
    cx.u_off = REC_U + 512 * TPW * slice;
#pragma unroll
    for (int d = 0; d < LEAD; ++d)
        if (d < NT)
            issue_chunk_split<TPW>(cx.rs, (uint32_t)d * REC_BYTES, (lds_u8*)L::ring() + d * L::SLOT,
                                   cx.u_off, cx.voff16);
    // chunks 0 and 1 (those that exist) before the first barrier
    wait_chunk<L::NL>(NT >= 2 ? min(LEAD, NT) - 2 : 0);
    copy_barrier();
    for (int c = 0; c < NT; c += RING) copy_round_split<0, TPW>(cx, c);
    copy_barrier();  // the output wave's last chunk
}

// Output wave, chunk c (slot S) after the barrier that ends chunk c + 1:
// for each tile, o = scale * (qg @ hc^T) + Aqk @ v_new (kernels.py:268-279)
// from the state wave's hand-off, as output_step forms it.
template <int S, int TPW>
__device__ __forceinline__ void output_step_split(const Ctx& cx, int c) {
    using L = SplitLds<TPW>;
    chunk_barrier();
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t* slot = L::ring() + S * L::SLOT;
    // Aqk 16 bytes at a time (this lane's 8 and its neighbour's), as in output_step
    const u32x4 aq2 = *reinterpret_cast<const u32x4*>(slot + REC_AQK + (cx.lane >> 1) * 16);
    const u32x2 aqk = (cx.lane & 1) ? u32x2{aq2.z, aq2.w} : u32x2{aq2.x, aq2.y};
    const int t = c * BT + 4 * cx.q4 + (cx.lane & 3);
    // every tile's hand-off read before the first store (no LDS read waits
    // behind a store)
    f32x4 qh[TPW];
    u32x2 vn[TPW];
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
        qh[i] = *reinterpret_cast<const f32x4*>(L::qh(S % HANDOFF, i) + cx.lane * 16);
        vn[i] = *reinterpret_cast<const u32x2*>(L::vn(S % HANDOFF, i) + cx.lane * 8);
    }
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
        f32x4 oacc = qh[i] * cx.scale;
        oacc = mfma_bf16_16x16x16(as_i16x4(aqk), as_i16x4(vn[i]), oacc);
        const u32x2 ot = quad_transpose(pack2(oacc[0], oacc[1]), pack2(oacc[2], oacc[3]), cx.lane & 3);
        if (t < cx.T)
            __builtin_nontemporal_store(
                ot, reinterpret_cast<u32x2*>(cx.obase + (int64_t)t * cx.orow_stride + 16 * i));
    }
}

template <int S, int TPW>
__device__ __forceinline__ void output_round_split(const Ctx& cx, int c) {
    output_step_split<S, TPW>(cx, c);
    if constexpr (S + 1 < RING) {
        if (c + 1 < cx.NT) output_round_split<S + 1, TPW>(cx, c + 1);
    }
}

enum Role { STATE = 0, OUTPUT = 1, COPY = 2, OUTPUT2 = 3 };

// Every wave executes exactly NT + 2 barriers: one after the prologue, one
// ending each chunk, and one more for the output wave's last chunk (it runs
// two chunks behind the state wave).  Each role ends its wave itself: with no join of
// the roles' code paths, the compiler's wait analysis of one role never
// sees another role's memory operations.
//
// MODE K2_TRAIN: the recompute of the backward; the output wave stores the
// training buffers instead of o (output_step).  MODE K2_BWD: the backward's
// state-gradient chain (bwd_state_wave) over the backward records, in
// reverse chunk order, its dh' and dv_new stored like the training buffers.
// MODE K2_FWD_MS: the forward with several sequences per work-group
// (above); grid seq_groups * HV * 8.  MODE K2_TRAIN_O: a training forward
// that keeps its state for the backward: o and ht as K2_FWD (the same
// arithmetic, so bit for bit), and h and v_new as K2_TRAIN; the first
// store wave forms o.
enum K2Mode { K2_FWD = 0, K2_TRAIN = 1, K2_BWD = 2, K2_FWD_MS = 3, K2_TRAIN_O = 4 };

// The training modes run a fourth wave, OUTPUT2, the second store wave.
template <int MODE>
__global__ __launch_bounds__(MODE == K2_FWD || MODE == K2_FWD_MS ? 192 : 256) void k2_kernel(Params p) {
    constexpr bool STORE_TR = MODE == K2_TRAIN || MODE == K2_BWD || MODE == K2_TRAIN_O;
    const int lane = threadIdx.x & 63;
    const int role = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if constexpr (MODE == K2_FWD_MS) {
        // (group, value head, value tile), XCD aware as below
        const int G = p.seq_groups;
        const int ngh = G * p.HV;
        const int wg = blockIdx.x;
        const int lin = (wg & 7) * ngh + (wg >> 3);
        const int gh = lin >> 3;
        const int g = gh / p.HV;
        const int nseq = p.cu_seqlens ? p.N : p.B;
        MsCtx m;
        m.hv = gh - g * p.HV;
        m.n0 = (int)((int64_t)g * nseq / G);
        m.n1 = (int)((int64_t)(g + 1) * nseq / G);
        m.J = 0;
        for (int n = m.n0; n < m.n1; ++n) m.J += seq_span(p, n * p.HV + m.hv).nt;
        Ctx cx;
        cx.scale = p.scale;
        cx.lane = lane;
        cx.q4 = lane >> 4;
        cx.vt = lin & 7;
        cx.rev = 0;
        cx.NT = m.J;
        if (role == STATE) {
            state_wave_ms(p, cx, m);
        } else if (role == OUTPUT) {
            output_wave_ms(p, cx, m);
        } else {
            copy_wave_ms(p, cx, m);
        }
        __builtin_amdgcn_endpgm();
    }
    const int nbh = (p.cu_seqlens ? p.N : p.B) * p.HV;

    // Work-group -> (head, value tile), XCD aware: consecutive work-group ids
    // go to different XCDs round-robin, so the 8 tiles of one head get ids
    // of one residue class mod 8 and share that XCD's L2 for the records.
    const int wg = blockIdx.x;
    const int lin = (wg & 7) * nbh + (wg >> 3);
    const int bh = lin >> 3;  // (batch row or sequence) * HV + value head
    const int hv = bh - (bh / p.HV) * p.HV;
    const SeqSpan sp = seq_span(p, bh);

    Ctx cx;
    cx.scale = p.scale;
    cx.NT = sp.nt;
    cx.T = sp.len;
    cx.lane = lane;
    cx.q4 = lane >> 4;
    cx.vt = lin & 7;
    cx.rev = MODE == K2_BWD;
    cx.ut = 0;

    if (sp.nt == 0) {
        // An empty sequence: its final state is its initial state.  Every
        // role sees the same count, so no wave reaches a barrier.
        if (role == STATE) {
            f32x4 St[8];
            const int v = 16 * cx.vt + (lane & 15);
            const int64_t sb = (int64_t)bh * DK * DK;
            if constexpr (MODE == K2_BWD) {
                // the initial state's gradient is the final state's
                load_state_from(p.dht ? p.dht + sb : nullptr, p.h0_v_first != 0, v, cx.q4, St);
                store_state_to(p.dh0 ? p.dh0 + sb : nullptr, p.h0_v_first != 0, v, cx.q4, St);
            } else {
                load_state(p, sb, v, cx.q4, St);
                store_state(p, sb, v, cx.q4, St);
            }
        }
        __builtin_amdgcn_endpgm();
    }
    if (role == STATE) {
        if constexpr (MODE == K2_BWD) {
            bwd_state_wave(p, cx, bh);
        } else {
            state_wave(p, cx, bh);
        }
        __builtin_amdgcn_endpgm();
    }
    if (role == OUTPUT) {
        output_wave<STORE_TR, 0, !STORE_TR || MODE == K2_TRAIN_O>(p, cx, sp, hv);
        __builtin_amdgcn_endpgm();
    }
    if constexpr (STORE_TR) {
        if (role == OUTPUT2) {
            output_wave<STORE_TR, 1, false>(p, cx, sp, hv);
            __builtin_amdgcn_endpgm();
        }
    }
    // the recompute for the backward stores h and v_new, not o: no qg
    copy_wave<MODE == K2_TRAIN ? LOADS_NO_QG : LOADS_PER_CHUNK>(p, cx, sp);
    __builtin_amdgcn_endpgm();
}

// Work-group (sequence, value head, slice of TPW value tiles), XCD aware as
// in kda_k2w.hip: the grid is padded to a multiple of 8 * (8 / TPW), and
// the 8 / TPW slices of a head get consecutive ids of one residue class
// mod 8, so they share an XCD and its L2 for the records.  Waves 0 .. TPW-1
// are the state waves, TPW the output wave, TPW + 1 the copy wave.
template <int TPW>
__global__ __launch_bounds__(64 * (TPW + 2)) void k2s_kernel(Params p) {
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

    Ctx cx;
    cx.scale = p.scale;
    cx.NT = sp.nt;
    cx.T = sp.len;
    cx.lane = lane;
    cx.q4 = lane >> 4;
    cx.rev = 0;
    cx.ut = wave < TPW ? wave : 0;
    cx.vt = slice * TPW + cx.ut;

    if (sp.nt == 0) {
        // An empty sequence: its final state is its initial state, and no
        // wave reaches a barrier.
        if (wave < TPW) {
            f32x4 St[8];
            const int v = 16 * cx.vt + (lane & 15);
            const int64_t sb = (int64_t)bh * DK * DK;
            load_state(p, sb, v, cx.q4, St);
            store_state(p, sb, v, cx.q4, St);
        }
        __builtin_amdgcn_endpgm();
    }
    if (wave < TPW) {
        state_wave<TPW>(p, cx, bh);
        __builtin_amdgcn_endpgm();
    }
    if (wave == TPW) {
        cx.obase = p.o + (sp.tok0 * p.HV + hv) * DK + 16 * TPW * slice + 4 * ((lane & 15) >> 2);
        cx.orow_stride = (int64_t)p.HV * DK;
        chunk_barrier();
        chunk_barrier();
        for (int c = 0; c < cx.NT; c += RING) output_round_split<0, TPW>(cx, c);
        __builtin_amdgcn_endpgm();
    }
    copy_wave_split<TPW>(p, cx, sp, slice);
    __builtin_amdgcn_endpgm();
}

}  // namespace

// CUs of the current device (cached per device).
static int cu_count() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cached[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

hipError_t launch_k2(const Params& p, hipStream_t stream) {
    const int nseq = p.cu_seqlens ? p.N : p.B;
    const int64_t tiles = (int64_t)p.HV * 8;
    const int ncu = cu_count();
    // More (sequence, head, value tile) triples than CUs: several tiles per
    // work-group share one record stream.  Two tiles: a state wave per tile
    // (k2s_kernel, above; B=1 T=4096 H=40 forward 148 against 166 us with
    // kda_k2w.hip's compute waves, H=64 205 against 213 us).  Four or eight,
    // or a caller's k2_wave_tiles: kda_k2w.hip.
    if (const int tpw = k2_wide_tiles(p, ncu)) {
        if (tpw == 2 && p.k2_wave_tiles == 0) {
            const int64_t nbh = (int64_t)(p.cu_seqlens ? p.N : p.B) * p.HV;
            const int64_t padded = (nbh * 4 + 31) / 32 * 32;  // 4 slices a head, 8 XCDs
            hipLaunchKernelGGL(k2s_kernel<2>, dim3((unsigned)padded), dim3(64 * 4), 0, stream, p);
            return hipGetLastError();
        }
        return launch_k2_wide(p, tpw, stream);
    }
    if (nseq > 1 && nseq * tiles > ncu) {
        // several sequences per work-group, in as many groups as fill the
        // CUs once (at least one)
        Params q = p;
        q.seq_groups = (int)std::max<int64_t>(1, std::min<int64_t>(nseq, ncu / tiles));
        hipLaunchKernelGGL(k2_kernel<K2_FWD_MS>, dim3((unsigned)(q.seq_groups * tiles)), dim3(192), 0,
                           stream, q);
        return hipGetLastError();
    }
    const int64_t grid = nseq * tiles;
    hipLaunchKernelGGL(k2_kernel<K2_FWD>, dim3((unsigned)grid), dim3(192), 0, stream, p);
    return hipGetLastError();
}

int fwd_plan(const Params& p) { return fused_forward(p, cu_count()) ? 1 : 0; }

// Segments of the two-stage forward.  A fixed-length forward whose records
// outgrow the infinity cache runs stage 1 then stage 2 over consecutive
// ranges of chunks, each range's records taking the workspace in turn and
// stage 2 carrying the state from one range to the next: the same
// arithmetic as one pass (stage 2 resumes from a state bit for bit), with
// the records stage 2 reads written moments before.  Above 200 MB of
// records, about 150 MB of records a segment (each of at least 64 chunks;
// at most 64 segments, a bound on the launches only), whatever stage 2's
// value tiles per work-group.  Measured, forward µs: B=1 T=8192 H=32 for
// 1 / 2 / 4 segments 261 / 249 / 269; T=8192 H=16, 143 MB of records, 186 /
// 190 / 215; T=8192 H=20, 178 MB, 199 / 210 for 1 / 2; T=8192 H=24,
// 214 MB, 221 / 221; ~100 MB segments lose to ~150 MB ones at every shape
// tried (c2 263 against 247.5 µs); at four tiles per work-group, T=8192
// H=96 607 / 597 for 1 / 6 segments (612 / 625 for 1 / 4, ~214 MB each),
// T=8192 H=80 558 / 530 (1 / 5); at 2.28 GB of records (T=16384 H=128)
// 1498 / 1431 for 8 / 16.  Not with packed sequences or debug outputs.
constexpr int64_t SEGMENT_MIN_RECORD_BYTES = 200000000;
constexpr int64_t SEGMENT_RECORD_BYTES = 150000000;
constexpr int MAX_SEGMENTS = 64;
constexpr int MIN_SEGMENT_CHUNKS = 64;

int fwd_segments(const Params& p) {
    if (p.cu_seqlens || p.dbg_Aqk) return 1;
    const int64_t rec = (int64_t)p.B * p.HV * p.NT * REC_BYTES;
    if (rec <= SEGMENT_MIN_RECORD_BYTES) return 1;
    int64_t n = (rec + SEGMENT_RECORD_BYTES - 1) / SEGMENT_RECORD_BYTES;
    n = std::min<int64_t>(n, MAX_SEGMENTS);
    n = std::min<int64_t>(n, p.NT / MIN_SEGMENT_CHUNKS);
    return (int)std::max<int64_t>(n, 1);
}

namespace {
// Stage 1 then stage 2 (the two launchers) over the forward's segments.
template <typename K1, typename K2>
hipError_t run_segments(const Params& p, int nseg, hipStream_t stream, K1 stage1, K2 stage2) {
    if (nseg == 1) {
        const hipError_t e = stage1(p, stream);
        return e != hipSuccess ? e : stage2(p, stream);
    }
    // Segment s: chunks [NT*s/nseg, NT*(s+1)/nseg).  Its records take the
    // front of the workspace; the state between segments (V-first) follows
    // them, which the workspace of the whole forward always has room for
    // (at least 64 chunks of records per (row, value head) are left over,
    // against 64 KiB of state).  A training forward's saved-state slots stay
    // the whole forward's (srec_stride, srec_off).
    const int64_t pairs = (int64_t)p.B * p.HV;
    const int64_t seg_chunks = (p.NT + nseg - 1) / nseg;
    float* state = reinterpret_cast<float*>(
        p.ws + ((pairs * seg_chunks * REC_BYTES + 255) / 256) * 256);  // segment_bytes
    const int gb = p.g_bf16 ? 2 : 4, bb = p.beta_bf16 ? 2 : 4;
    for (int s = 0; s < nseg; ++s) {
        const int c0 = (int)((int64_t)p.NT * s / nseg), c1 = (int)((int64_t)p.NT * (s + 1) / nseg);
        const int64_t t0 = (int64_t)c0 * BT;
        Params q = p;
        q.T = (int)std::min<int64_t>(p.T - t0, (int64_t)(c1 - c0) * BT);
        q.NT = c1 - c0;
        q.srec_stride = p.NT;
        q.srec_off = c0;
        q.q = p.q + t0 * p.H * DK;
        q.k = p.k + t0 * p.H * DK;
        q.v = p.v + t0 * p.HV * DK;
        q.g = static_cast<const uint8_t*>(p.g) + t0 * p.HV * DK * gb;
        q.beta = static_cast<const uint8_t*>(p.beta) + t0 * p.HV * bb;
        q.o = p.o + t0 * p.HV * DK;
        if (s > 0) {
            q.h0 = state;
            q.h0_v_first = 1;
        }
        if (s + 1 < nseg) {
            q.ht = state;
            q.ht_v_first = 1;
        }
        hipError_t e = stage1(q, stream);
        if (e == hipSuccess) e = stage2(q, stream);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}
}  // namespace

hipError_t launch_two_stage(const Params& p, hipStream_t stream) {
    return run_segments(p, fwd_segments(p), stream, launch_k1, launch_k2);
}

// Workspace bytes of a fixed-length forward in nseg > 1 segments: one
// segment's records, then the state carried between segments.
int64_t segment_bytes(const Params& p, int nseg) {
    const int64_t pairs = (int64_t)p.B * p.HV;
    const int64_t seg_chunks = (p.NT + nseg - 1) / nseg;
    return (pairs * seg_chunks * REC_BYTES + 255) / 256 * 256 + pairs * DK * DK * 4;
}

// The fewest segments, at least fwd_segments' count, whose workspace fits
// max_bytes (segments as short as one chunk), or 0 when none does or the
// forward cannot run in segments (packed sequences, debug outputs).
int segments_to_fit(const Params& p, int64_t max_bytes) {
    if (p.cu_seqlens || p.dbg_Aqk) return 0;
    for (int n = std::max(2, fwd_segments(p)); n <= p.NT; ++n)
        if (segment_bytes(p, n) <= max_bytes) return n;
    return 0;
}

hipError_t launch_two_stage_in(const Params& p, int nseg, hipStream_t stream) {
    return run_segments(p, nseg, stream, launch_k1, launch_k2);
}

// The training forward (kda_bt16_fwd_save_hip): o and ht as launch_two_stage,
// plus the state the backward starts from.
hipError_t launch_fwd_save(const Params& p, hipStream_t stream) {
    return run_segments(p, fwd_segments(p), stream, launch_k1_save, launch_k2_train_o);
}

hipError_t launch_k2_train(const Params& p, hipStream_t stream) {
    const int64_t grid = (int64_t)(p.cu_seqlens ? p.N : p.B) * p.HV * 8;
    hipLaunchKernelGGL(k2_kernel<K2_TRAIN>, dim3((unsigned)grid), dim3(256), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_k2_train_o(const Params& p, hipStream_t stream) {
    const int64_t grid = (int64_t)(p.cu_seqlens ? p.N : p.B) * p.HV * 8;
    hipLaunchKernelGGL(k2_kernel<K2_TRAIN_O>, dim3((unsigned)grid), dim3(256), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_k2_bwd(const Params& p, hipStream_t stream) {
    const int64_t grid = (int64_t)(p.cu_seqlens ? p.N : p.B) * p.HV * 8;
    hipLaunchKernelGGL(k2_kernel<K2_BWD>, dim3((unsigned)grid), dim3(256), 0, stream, p);
    return hipGetLastError();
}

}  // namespace kda
