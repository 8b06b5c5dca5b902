// The compute step of the wide stage 2 (kda_k2w.hip), shared with the
// fused forward (kda_fused.hip): one compute wave's chunk of the recurrence
// (kernels.py:225-302) for one or two 16-column value tiles, with its
// operands read from a record in LDS, in kda_k2.hip's arithmetic.
#pragma once

#include "kda_common.h"
#include "kda_k2_shared.h"

namespace kda {
namespace {

// The operands a compute wave reads for one chunk.
struct WideOps {
    u32x4 w[4];   // -w, 16x16x32 A operands (k-tile pairs)
    u32x4 qg[4];  // qg, likewise
    u32x4 kg[4];  // kg, 16x16x16 A operands of the update (two k-tiles each)
    u32x2 aqk;    // Aqk, 16x16x16 A operand
    f32x2 dc;     // 2^G_last for the decay broadcast
};

__device__ __forceinline__ void read_wide_ops(const uint8_t* slot, int lane, int ut, WideOps& op) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        op.w[j] = *reinterpret_cast<const u32x4*>(slot + REC_W + j * 1024 + lane * 16);
        op.qg[j] = *reinterpret_cast<const u32x4*>(slot + REC_QG + j * 1024 + lane * 16);
        op.kg[j] = *reinterpret_cast<const u32x4*>(slot + REC_KG + j * 1024 + lane * 16);
    }
    op.aqk = *reinterpret_cast<const u32x2*>(slot + REC_AQK + lane * 8);
    op.dc = *reinterpret_cast<const f32x2*>(slot + decay_offset(lane));
}

__device__ __forceinline__ f32x4 unpack_u(u32x2 u) {
    return f32x4{__builtin_bit_cast(float, u.x << 16), __builtin_bit_cast(float, u.x & 0xffff0000u),
                 __builtin_bit_cast(float, u.y << 16), __builtin_bit_cast(float, u.y & 0xffff0000u)};
}

// bf16(S^T) of k-tiles 2j, 2j+1 of one value tile: a 16x16x32 B operand.
__device__ __forceinline__ u32x4 pack_hc(const f32x4 (&St)[8], int j) {
    return u32x4{pack2(St[2 * j][0], St[2 * j][1]), pack2(St[2 * j][2], St[2 * j][3]),
                 pack2(St[2 * j + 1][0], St[2 * j + 1][1]),
                 pack2(St[2 * j + 1][2], St[2 * j + 1][3])};
}

// k-tile KT of both tiles' state update: S = S * 2^G_last + kg^T v_new (the
// decay a VALU product on the accumulator input, as kda_k2.hip forms it).
template <int KT>
__device__ __forceinline__ void wide_update(f32x4 (&SA)[8], f32x4 (&SB)[8], const WideOps& op,
                                            u32x2 vna, u32x2 vnb) {
    const u32x4 kg = op.kg[KT >> 1];
    const i16x4 a = as_i16x4((KT & 1) ? u32x2{kg.z, kg.w} : u32x2{kg.x, kg.y});
    SA[KT] = mfma_bf16_16x16x16(a, as_i16x4(vna), decay_tile<KT>(SA[KT], op.dc));
    SB[KT] = mfma_bf16_16x16x16(a, as_i16x4(vnb), decay_tile<KT>(SB[KT], op.dc));
}

// Constants of a compute wave.
struct WideCtx {
    uint16_t* obase[2];   // o of the sequence's first token, this lane's 4 columns of each tile
    int64_t orow_stride;  // elements between consecutive tokens of o
    float scale;
    int NT, T, lane, q4;
};

// How the waves of a work-group meet around one chunk of a compute wave:
// `ready(c)` before the wave reads chunk c's operands from their ring slot,
// `consumed()` once those reads are issued, `end()` after the chunk; and
// where u comes from: `read_u` with the slot reads, `u_start(t)` for tile
// t's accumulator start after them.  kda_k2w.hip: one barrier per chunk,
// u as stage 1 stored it (BarrierHooks); kda_fused.hip: LDS flags between
// the waves that form the records and those that read them, u formed here
// from the operands the producers leave in its place.
struct BarrierHooks {
    u32x2 u[2];  // u of the two tiles (bf16 pairs)
    __device__ __forceinline__ void ready(int) {}
    __device__ __forceinline__ void read_u(const uint8_t* slot, int lane, int ut) {
        u[0] = *reinterpret_cast<const u32x2*>(slot + REC_SHARED + ut * 512 + lane * 8);
        u[1] = *reinterpret_cast<const u32x2*>(slot + REC_SHARED + (ut + 1) * 512 + lane * 8);
    }
    __device__ __forceinline__ void consumed() {}
    __device__ __forceinline__ f32x4 u_start(int t) const { return unpack_u(u[t]); }
    __device__ __forceinline__ void end() { chunk_barrier(); }
};

// One chunk of a compute wave: both tiles' v_new, o and state update, with
// chunk c's operands read from its ring slot at the start.  The reads are
// covered by the packing of hc, which needs only the state; one operand set
// is live at a time.
template <class Hooks>
__device__ __forceinline__ void wide_step(const WideCtx& cx, int c, f32x4 (&SA)[8], f32x4 (&SB)[8],
                                          const uint8_t* slot, int ut, Hooks& hk) {
    hk.ready(c);
    WideOps cur;
    read_wide_ops(slot, cx.lane, ut, cur);
    hk.read_u(slot, cx.lane, ut);
    u32x4 ha[4], hb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        ha[j] = pack_hc(SA, j);
        hb[j] = pack_hc(SB, j);
    }
    hk.consumed();
    // v_new = u - w @ hc^T: one accumulation chain per tile, from u
    f32x4 va = hk.u_start(0);
    f32x4 vb = hk.u_start(1);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        va = mfma_bf16_16x16x32(as_bf16x8(cur.w[j]), as_bf16x8(ha[j]), va);
        vb = mfma_bf16_16x16x32(as_bf16x8(cur.w[j]), as_bf16x8(hb[j]), vb);
    }
    // o = scale * qg @ hc^T + Aqk @ v_new
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    f32x4 oa = zero, ob = zero;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        oa = mfma_bf16_16x16x32(as_bf16x8(cur.qg[j]), as_bf16x8(ha[j]), oa);
        ob = mfma_bf16_16x16x32(as_bf16x8(cur.qg[j]), as_bf16x8(hb[j]), ob);
    }
    const u32x2 vna = {pack2(va[0], va[1]), pack2(va[2], va[3])};
    const u32x2 vnb = {pack2(vb[0], vb[1]), pack2(vb[2], vb[3])};
    oa = oa * cx.scale;
    ob = ob * cx.scale;
    oa = mfma_bf16_16x16x16(as_i16x4(cur.aqk), as_i16x4(vna), oa);
    ob = mfma_bf16_16x16x16(as_i16x4(cur.aqk), as_i16x4(vnb), ob);
    // state update: S = S * 2^G_last + kg^T v_new, tile by tile
    wide_update<0>(SA, SB, cur, vna, vnb);
    wide_update<1>(SA, SB, cur, vna, vnb);
    wide_update<2>(SA, SB, cur, vna, vnb);
    wide_update<3>(SA, SB, cur, vna, vnb);
    wide_update<4>(SA, SB, cur, vna, vnb);
    wide_update<5>(SA, SB, cur, vna, vnb);
    wide_update<6>(SA, SB, cur, vna, vnb);
    wide_update<7>(SA, SB, cur, vna, vnb);
    // Lane (x, q4) holds o rows 4*q4 .. +3 of column x; after the quad
    // transpose it holds row 4*q4 + x%4, columns 4*(x/4) .. +3.
    const int j4 = cx.lane & 3;
    const u32x2 ota = quad_transpose(pack2(oa[0], oa[1]), pack2(oa[2], oa[3]), j4);
    const u32x2 otb = quad_transpose(pack2(ob[0], ob[1]), pack2(ob[2], ob[3]), j4);
    // Ordinary stores: the 8-byte pieces of one 256-byte row of o come from
    // different waves, and merge in L2 (non-temporal stores of the same
    // pieces made stage 2 ~10% slower at B=1 T=8192 H=96).
    const int t = c * BT + 4 * cx.q4 + j4;
    if (t < cx.T) {
        const int64_t off = (int64_t)t * cx.orow_stride;
        *reinterpret_cast<u32x2*>(cx.obase[0] + off) = ota;
        *reinterpret_cast<u32x2*>(cx.obase[1] + off) = otb;
    }
    hk.end();
}

// k-tile KT of a single tile's state update (TW = 1).
template <int KT>
__device__ __forceinline__ void wide1_update(f32x4 (&S)[8], const u32x4 (&kg)[4], f32x2 dc, u32x2 vn) {
    const u32x4 k2 = kg[KT >> 1];
    const i16x4 a = as_i16x4((KT & 1) ? u32x2{k2.z, k2.w} : u32x2{k2.x, k2.y});
    S[KT] = mfma_bf16_16x16x16(a, as_i16x4(vn), decay_tile<KT>(S[KT], dc));
}

// One chunk of a compute wave that owns a single value tile (TW = 1): the
// arithmetic of wide_step for one of its tiles.
__device__ __forceinline__ void wide1_step(const WideCtx& cx, int c, f32x4 (&S)[8], const uint8_t* slot,
                                           int ut) {
    u32x4 w[4], qg[4], kg[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        w[j] = *reinterpret_cast<const u32x4*>(slot + REC_W + j * 1024 + cx.lane * 16);
        qg[j] = *reinterpret_cast<const u32x4*>(slot + REC_QG + j * 1024 + cx.lane * 16);
        kg[j] = *reinterpret_cast<const u32x4*>(slot + REC_KG + j * 1024 + cx.lane * 16);
    }
    const u32x2 aqk = *reinterpret_cast<const u32x2*>(slot + REC_AQK + cx.lane * 8);
    const f32x2 dc = *reinterpret_cast<const f32x2*>(slot + decay_offset(cx.lane));
    const u32x2 u = *reinterpret_cast<const u32x2*>(slot + REC_SHARED + ut * 512 + cx.lane * 8);
    u32x4 hc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) hc[j] = pack_hc(S, j);
    // v_new = u - w @ hc^T, one accumulation chain from u
    f32x4 v = unpack_u(u);
#pragma unroll
    for (int j = 0; j < 4; ++j) v = mfma_bf16_16x16x32(as_bf16x8(w[j]), as_bf16x8(hc[j]), v);
    // o = scale * qg @ hc^T + Aqk @ v_new
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    f32x4 o = zero;
#pragma unroll
    for (int j = 0; j < 4; ++j) o = mfma_bf16_16x16x32(as_bf16x8(qg[j]), as_bf16x8(hc[j]), o);
    const u32x2 vn = {pack2(v[0], v[1]), pack2(v[2], v[3])};
    o = o * cx.scale;
    o = mfma_bf16_16x16x16(as_i16x4(aqk), as_i16x4(vn), o);
    wide1_update<0>(S, kg, dc, vn);
    wide1_update<1>(S, kg, dc, vn);
    wide1_update<2>(S, kg, dc, vn);
    wide1_update<3>(S, kg, dc, vn);
    wide1_update<4>(S, kg, dc, vn);
    wide1_update<5>(S, kg, dc, vn);
    wide1_update<6>(S, kg, dc, vn);
    wide1_update<7>(S, kg, dc, vn);
    const int j4 = cx.lane & 3;
    const u32x2 ot = quad_transpose(pack2(o[0], o[1]), pack2(o[2], o[3]), j4);
    const int t = c * BT + 4 * cx.q4 + j4;
    if (t < cx.T) *reinterpret_cast<u32x2*>(cx.obase[0] + (int64_t)t * cx.orow_stride) = ot;
    chunk_barrier();
}

}  // namespace
}  // namespace kda
