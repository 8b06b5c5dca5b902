// Stage 1's per-chunk work: everything of one (sequence, value head,
// 16-token chunk) that does not depend on the recurrent state, formed by one
// 64-lane wave and written as the chunk's 17 KiB record.  Shared by the
// stage-1 kernels (kda_k1.hip), which write the record to the workspace in
// HBM, and the fused forward (kda_fused.hip), which writes it into an LDS
// ring that its state waves read.
//
// Follows kda_bt16_kernel_k1 (/root/reference/src/kda_bt16/kernels.py:53-184);
// the lane layout is described in kda_k1.hip.
#pragma once

#include "kda_common.h"

namespace kda {
namespace {

// 32 bf16 values of one row in F order, packed: item 4*kt + i is half
// (i & 1) of word (i >> 1) of v[kt].
struct Row32 {
    u32x2 v[8];
};

__device__ __forceinline__ float elem(const Row32& a, int p) {
    const uint32_t w = (p & 2) ? a.v[p >> 2].y : a.v[p >> 2].x;
    return (p & 1) ? __builtin_bit_cast(float, w & 0xffff0000u) : __builtin_bit_cast(float, w << 16);
}

__device__ __forceinline__ void load_row(const uint16_t* __restrict__ src, bool valid, int colbase,
                                         Row32& out) {
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
        out.v[kt] = u32x2{0u, 0u};
        if (valid) out.v[kt] = *reinterpret_cast<const u32x2*>(src + 16 * kt + colbase);
    }
}

__device__ __forceinline__ u32x2 pack4(float a, float b, float c, float d) {
    return u32x2{pack2(a, b), pack2(c, d)};
}
__device__ __forceinline__ u32x2 pack4(f32x4 v) { return pack4(v.x, v.y, v.z, v.w); }

// The 16x16x16 B operand of the identity: lane (n, q4) holds
// I[4*q4 + i][n], bf16 1.0 where 4*q4 + i = n.
__device__ __forceinline__ i16x4 eye_operand(int lane) {
    const int n = lane & 15, k0 = 4 * (lane >> 4);
    constexpr short ONE = 0x3F80;
    return i16x4{short(k0 == n ? ONE : 0), short(k0 + 1 == n ? ONE : 0), short(k0 + 2 == n ? ONE : 0),
                 short(k0 + 3 == n ? ONE : 0)};
}

// Tile kt of a 16x128 bf16 matrix M from F order to T order, through the
// matrix core: F order, lane (r, q4) holding M[r][16*kt + 4*q4 + i], is the
// 16x16x16 A layout, so D = M @ I lands as D[4*q4 + i][r], i.e. T order,
// lane (r, q4) holding M[4*q4 + i][16*kt + r] (the layout of a 16x16x16 B
// operand, or an A operand of M^T).  Exact: every sum holds one product,
// x * 1.
__device__ __forceinline__ i16x4 tile_T(u32x2 f, i16x4 eye) {
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    return as_i16x4(pack4(mfma_bf16_16x16x16(as_i16x4(f), eye, zero)));
}

// Tile vt of u = bf16(A @ bf16(v * beta)) (kernels.py:173-174) from the raw
// v tile in F order (lane (r, q4) holding v[r][16*vt + 4*q4 + i]), the
// lane's row's beta and bf16(A_inv) as the 16x16x16 A operand; it lands as
// u[4*q4 + i][16*vt + r], the order stage 2 subtracts it in.  Stage 1 and
// the fused forward's compute waves both form u with it.
__device__ __forceinline__ u32x2 form_u(u32x2 v, float beta, i16x4 A_op, i16x4 eye) {
    const float v0 = __builtin_bit_cast(float, v.x << 16);
    const float v1 = __builtin_bit_cast(float, v.x & 0xffff0000u);
    const float v2 = __builtin_bit_cast(float, v.y << 16);
    const float v3 = __builtin_bit_cast(float, v.y & 0xffff0000u);
    const i16x4 vbT = tile_T(pack4(v0 * beta, v1 * beta, v2 * beta, v3 * beta), eye);
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    return pack4(mfma_bf16_16x16x16(A_op, vbT, zero));
}

// LDS scratch of one wave's k1_chunk: L and the solve's columns (fp32), in
// bytes.
constexpr int K1_SCRATCH_L = BT * BT * 4;
constexpr int K1_SCRATCH_X = BT * (BT + 1) * 4;
constexpr int K1_SCRATCH = K1_SCRATCH_L + K1_SCRATCH_X;

// The wave's own LDS writes are complete before its next LDS read: the
// scratch of k1_chunk belongs to one wave, so no work-group barrier is
// needed between its phases.
__device__ __forceinline__ void wave_lds_fence() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Record modes.  K1_FWD: the forward record.  K1_BOTH (the backward's
// recompute): the forward record without qg (no o is formed), the gram
// block in qg's bytes, and the backward record with dO.  K1_SAVE (a
// training forward that keeps its state for the backward): the forward
// record, the gram block, and the backward record without dO, which the
// backward adds (k1_dout_kernel) once dO exists.
enum K1Mode { K1_FWD = 0, K1_BOTH = 1, K1_SAVE = 2 };

// The fused forward's ring slot (kda_fused.hip): the forward record with
// u left to the compute waves, whose producers have the scarcer issue
// slots.  In u's place the slot holds the chunk's raw v tiles in the
// order u would take ([vt][lane][4] bf16, F order: lane (r, q4) holds
// v[r][16*vt + 4*q4 + i]); then bf16(A_inv) as the 16x16x16 A operand
// ([lane][4]) and beta per row as stage 1 applied it (fp32 [16]).  The
// compute waves form u = bf16(A @ bf16(v * beta)) with the instructions
// stage 1 uses (form_u), so u is the same bits.
constexpr int FREC_A = REC_BYTES;
constexpr int FREC_BETA = REC_BYTES + 512;
constexpr int FREC_BYTES = REC_BYTES + 1024;

// The inputs of one chunk: k1_load issues their loads, k1_compute uses
// them, so that a caller can load the next chunk while it works on this one
// (the fused forward's producer waves).  Members a mode does not use are
// never set.
template <bool GB16, bool WITH_DO>
struct K1In {
    Row32 q, k, v;
    Row32 dout;          // the backward's dO rows (WITH_DO)
    Row32 g16;           // g as bf16 (GB16)
    f32x4 g32[8];        // g as fp32
    uint32_t beta_bits;  // raw: bf16 in the low half, or fp32
};

// The lane's row of chunk c and where it lies.
struct K1Row {
    int lane, r, q4, colbase, h, t0, nvalid;
    bool valid;
    int64_t tok, rowoff, vrowoff;
};

template <bool FULL>
__device__ __forceinline__ K1Row k1_row(const Params& p, int hv, int c, const SeqSpan& sp) {
    K1Row w;
    w.lane = threadIdx.x & 63;  // the wave's lane (several waves in the fused forward)
    w.r = w.lane & 15;
    w.q4 = w.lane >> 4;
    w.colbase = 4 * w.q4;
    w.h = hv / (p.HV / p.H);  // the q/k head of this value head
    w.t0 = c * BT;
    w.nvalid = FULL ? BT : min(BT, sp.len - w.t0);
    w.valid = FULL || w.r < w.nvalid;
    w.tok = sp.tok0 + w.t0 + w.r;                 // token of this lane's row
    w.rowoff = (w.tok * p.H + w.h) * DK;          // q/k element offset of that row
    w.vrowoff = (w.tok * p.HV + hv) * DK;         // v/g element offset of that row
    return w;
}

// ---- loads (kernels.py:97-106); padded rows read as zero -----------------
// Every load of the chunk is issued before the first wait: values are
// converted only where they are used, and optional operands are read
// through a pointer select (kZeroCols when absent) rather than behind a
// branch, so that no load waits for another's round trip.
template <int K1M, bool FULL, bool GB16>
__device__ __forceinline__ void k1_load(const Params& p, int hv, int c, const SeqSpan& sp,
                                        K1In<GB16, K1M == K1_BOTH>& in) {
    const K1Row w = k1_row<FULL>(p, hv, c, sp);
    load_row(p.q + w.rowoff, w.valid, w.colbase, in.q);
    load_row(p.k + w.rowoff, w.valid, w.colbase, in.k);
    load_row(p.v + w.vrowoff, w.valid, w.colbase, in.v);
    if constexpr (K1M == K1_BOTH) load_row(p.dout + w.vrowoff, w.valid, w.colbase, in.dout);
    if constexpr (GB16) {
        load_row(static_cast<const uint16_t*>(p.g) + w.vrowoff, w.valid, w.colbase, in.g16);
    } else {
        const float* gsrc = static_cast<const float*>(p.g) + w.vrowoff;
#pragma unroll
        for (int kt = 0; kt < 8; ++kt) {
            in.g32[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (w.valid) in.g32[kt] = *reinterpret_cast<const f32x4*>(gsrc + 16 * kt + w.colbase);
        }
    }
    in.beta_bits = 0u;
    if (w.valid) {
        const int64_t bi = w.tok * p.HV + hv;
        if (p.beta_bf16) in.beta_bits = static_cast<const uint16_t*>(p.beta)[bi];
        else in.beta_bits = static_cast<const uint32_t*>(p.beta)[bi];
    }
}

// The head's 128 dt_bias values (global or LDS), or kZeroCols without them.
__device__ __forceinline__ const float* k1_bias(const Params& p, int hv) {
    return p.use_gate && p.dt_bias ? p.dt_bias + hv * DK : kZeroCols;
}

// exp(A_log) of the head (1 without the in-kernel gate).
__device__ __forceinline__ float k1_ea(const Params& p, int hv) {
    float ea = expf(*(p.use_gate ? p.A_log + hv : kZeroCols));
    asm volatile("" : "+v"(ea));  // formed here, not sunk to its use
    return ea;
}

// The work on one chunk's inputs: biasp the head's dt_bias (k1_bias, or a
// copy of it), ea = k1_ea.
template <int K1M, bool FULL, bool GB16, bool U_IN_SLOT = false>
__device__ __forceinline__ void k1_compute(const Params& p, int hv, int c, const SeqSpan& sp,
                                           const K1In<GB16, K1M == K1_BOTH>& in, const float* biasp,
                                           float ea, float* sL, float* sX, uint8_t* rec) {
    constexpr bool BOTH = K1M != K1_FWD;
    constexpr bool WITH_DO = K1M == K1_BOTH;
    const K1Row w = k1_row<FULL>(p, hv, c, sp);
    const int lane = w.lane, r = w.r, q4 = w.q4, colbase = w.colbase;
    const int HV = p.HV;
    const int t0 = w.t0;
    const int nvalid = w.nvalid;
    const bool valid = w.valid;
    const int64_t tok = w.tok;
    const int64_t vrowoff = w.vrowoff;
    Row32 qp = in.q, kp = in.k;
    const Row32& vp = in.v;
    const Row32& dop = in.dout;
    const Row32& gp = in.g16;
    const f32x4 (&gf)[8] = in.g32;
    f32x4 bias[8];  // zeros without dt_bias (k1_bias), so s = g + bias either way
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) bias[kt] = *reinterpret_cast<const f32x4*>(biasp + 16 * kt + colbase);
    const uint32_t beta_bits = in.beta_bits;
    float G[32];
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) G[4 * kt + i] = GB16 ? elem(gp, 4 * kt + i) : gf[kt][i];
    }
    float beta = __builtin_bit_cast(float, p.beta_bf16 ? beta_bits << 16 : beta_bits);
    if (p.use_beta_sigmoid) beta = fast_sigmoid(beta);

    // ---- q/k l2norm, rounded back to bf16 (kernels.py:108-113) -----------
    if (p.use_l2norm) {
        float sq = 0.f, sk = 0.f;
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            sq = fmaf(elem(qp, j), elem(qp, j), sq);
            sk = fmaf(elem(kp, j), elem(kp, j), sk);
        }
        sq += xor16(sq);
        sk += xor16(sk);
        sq += __shfl_xor(sq, 32);
        sk += __shfl_xor(sk, 32);
        const float rq = 1.f / sqrtf(sq + L2_EPS);
        const float rk = 1.f / sqrtf(sk + L2_EPS);
#pragma unroll
        for (int kt = 0; kt < 8; ++kt) {
            qp.v[kt] = pack4(elem(qp, 4 * kt) * rq, elem(qp, 4 * kt + 1) * rq,
                             elem(qp, 4 * kt + 2) * rq, elem(qp, 4 * kt + 3) * rq);
            kp.v[kt] = pack4(elem(kp, 4 * kt) * rk, elem(kp, 4 * kt + 1) * rk,
                             elem(kp, 4 * kt + 2) * rk, elem(kp, 4 * kt + 3) * rk);
        }
    }

    // ---- gate and chunk-local log2 cumsum (kernels.py:115-124) -----------
    // sigmoid(ea * s) = 1 / (1 + 2^(s * ea * -log2 e)), with ea * -log2 e
    // formed once; the cumsum is linear, so lower_bound joins the 1/ln 2
    // after it (one product per element each, not three).
    if (p.use_gate) {
        const float eal = ea * -1.4426950408889634f;
        const float lbr = p.lower_bound * RCP_LN2;
#pragma unroll
        for (int kt = 0; kt < 8; ++kt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float s = G[4 * kt + i] + bias[kt][i];
                float sig = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(s * eal));
                sig = valid ? sig : 0.f;
                G[4 * kt + i] = row_scan16(sig) * lbr;
            }
        }
    } else if (p.g_log) {
        // g is the per-token natural-log decay: the same cumsum-then-scale
        // as the in-kernel gate, on g itself.
#pragma unroll
        for (int j = 0; j < 32; ++j) G[j] = row_scan16(valid ? G[j] : 0.f) * RCP_LN2;
    }

    // ---- mid-row recentring, grams on matrix cores (kernels.py:129-155) ---
    const int mid = min(BT / 2, nvalid - 1);
    const int last = nvalid - 1;
    const int row0 = lane & 48;
    // Row mid's and row last's values reach the rows of their 16-lane
    // group by DPP broadcast in a full chunk (mid = 8, last = 15), by a
    // cross-lane permute in a sequence's partial last chunk.
    auto bcast_mid = [&](auto use) {
        if constexpr (FULL) use([](float x) { return row_bcast<BT / 2>(x); });
        else use([&](float x) { return shfl(x, row0 | mid); });
    };
    auto bcast_last = [&](auto use) {
        if constexpr (FULL) use([](float x) { return row_bcast<BT - 1>(x); });
        else use([&](float x) { return shfl(x, row0 | last); });
    };
    f32x4 acc_qk = {0.f, 0.f, 0.f, 0.f};
    f32x4 acc_kk = {0.f, 0.f, 0.f, 0.f};
    bcast_mid([&](auto from_mid) {
#pragma unroll
        for (int j = 0; j < 32; ++j) {
            const float gm = G[j] - from_mid(G[j]);
            const float gq = valid ? fast_exp2(gm) : 0.f;
            const float gk = valid ? fast_exp2(-gm) : 0.f;
            const float qv = elem(qp, j), kv = elem(kp, j);
            // A = Ks (rows s), B = Qs / Kq (columns t): lane (t, q4) receives
            // Aqk[t][4*q4 + i] and Akk[t][4*q4 + i].
            acc_qk = mfma_f32_16x16x4(kv * gk, qv * gq, acc_qk);
            acc_kk = mfma_f32_16x16x4(kv * gk, kv * gq, acc_kk);
        }
    });

    // This chunk's record goes to `rec` with ordinary stores: in the
    // workspace, the grid runs the chunks last to first (k1_kernel), so the
    // records stage 2 reads first are the ones written last, still in L2 and
    // the infinity cache; in the fused forward, `rec` is a ring slot in LDS.
    // (The backward record below is streamed out with non-temporal stores.)

    f32x4 aqk, L;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int s = 4 * q4 + i;
        aqk[i] = (r >= s) ? acc_qk[i] * p.scale : 0.f;
        L[i] = (r > s) ? acc_kk[i] * beta : 0.f;
    }
    const u32x2 aqk_bf = pack4(aqk);
    *reinterpret_cast<u32x2*>(rec + REC_AQK + lane * 8) = aqk_bf;

    // ---- (I + L)^-1 by forward substitution (kernels.py:157-167) ---------
    // Lane r solves column s = r: a[t] = A_inv[t][s], with a[s] = 1,
    // a[t < s] = 0 and a[t > s] = -sum_{j<t} L[t][j] a[j].
    *reinterpret_cast<f32x4*>(sL + r * BT + 4 * q4) = L;
    wave_lds_fence();
    {
        float a[BT];
#pragma unroll
        for (int t = 0; t < BT; ++t) {
            float acc = 0.f;
#pragma unroll
            for (int j4 = 0; j4 < (t + 3) / 4; ++j4) {
                const f32x4 lr = *reinterpret_cast<const f32x4*>(sL + t * BT + 4 * j4);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if (4 * j4 + i < t) acc = fmaf(-lr[i], a[4 * j4 + i], acc);
                }
            }
            // above the diagonal (t < r) every a[j < t] is zero, so acc is
            // +0 there
            a[t] = t == r ? 1.f : acc;
        }
        if (q4 == 0) {
#pragma unroll
            for (int t = 0; t < BT; ++t) sX[r * (BT + 1) + t] = a[t];
        }
    }
    wave_lds_fence();
    f32x4 ainv;
#pragma unroll
    for (int i = 0; i < 4; ++i) ainv[i] = sX[(4 * q4 + i) * (BT + 1) + r];
    const u32x2 ainv_bf = pack4(ainv);  // A = bf16(A_inv), kernels.py:170
    if constexpr (BOTH) {
        // the gram and the inverse for the per-chunk gradients (kda_common.h)
        uint8_t* la = p.la + (sp.srec0 + c) * p.la_stride;
        __builtin_nontemporal_store(acc_kk, reinterpret_cast<f32x4*>(la + LA_LRAW + lane * 16));
        __builtin_nontemporal_store(ainv, reinterpret_cast<f32x4*>(la + LA_AINV + lane * 16));
    }
    const i16x4 A_op = as_i16x4(ainv_bf);
    const i16x4 A_neg = as_i16x4(ainv_bf ^ 0x80008000u);
    // the identity operand of the transposes through the matrix core (tile_T)
    const i16x4 eye = eye_operand(lane);

    if constexpr (BOTH) {
        // ---- backward record ---------------------------------------------
        uint8_t* brec = p.ws_bwd + (sp.srec0 + c) * REC_BYTES;
        // Aqk^T as an A operand: lane (r, q4) takes Aqk[4*q4 + i][r], the
        // transpose of what it holds (bf16 rounding commutes with it).
        __builtin_nontemporal_store(__builtin_bit_cast(u32x2, tile_T(aqk_bf, eye)),
                                    reinterpret_cast<u32x2*>(brec + BREC_AQKT + lane * 8));
        // -w in T order straight from the matrix cores: (-A) @ kb tile kt
        // lands as -w[4*q4 + i][16*kt + r]; bf16(scale * q^ * 2^G) in T
        // order.
#pragma unroll
        for (int kt = 0; kt < 8; ++kt) {
            float kb[4], qs[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float e = fast_exp2(G[4 * kt + i]);
                kb[i] = round_bf(elem(kp, 4 * kt + i) * beta) * e;
                qs[i] = p.scale * (elem(qp, 4 * kt + i) * e);
            }
            const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
            const u32x2 wT = pack4(mfma_bf16_16x16x16(A_neg, tile_T(pack4(kb[0], kb[1], kb[2], kb[3]), eye), zero));
            const u32x2 qv = __builtin_bit_cast(u32x2, tile_T(pack4(qs[0], qs[1], qs[2], qs[3]), eye));
            __builtin_nontemporal_store(u32x4{qv.x, qv.y, wT.x, wT.y},
                                        reinterpret_cast<u32x4*>(brec + BREC_UPD + kt * 1024 + lane * 16));
        }
        // dO as the B operand of each value tile (T order, the layout of u
        // in the forward record): [vt][lane][i] = dO[4*q4 + i][16*vt + r].
        if constexpr (WITH_DO) {
#pragma unroll
            for (int vt = 0; vt < 8; ++vt)
                __builtin_nontemporal_store(__builtin_bit_cast(u32x2, tile_T(dop.v[vt], eye)),
                                            reinterpret_cast<u32x2*>(brec + BREC_DO + vt * 512 + lane * 8));
        }
        // kg = bf16(k^ * 2^(G_last - G)) in F order (the A operand of
        // kg @ dh), and the decay 2^G_last.
        u32x2 kgF[8];
        bcast_last([&](auto from_last) {
#pragma unroll
            for (int kt = 0; kt < 8; ++kt) {
                float kg[4], gl[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    gl[i] = from_last(G[4 * kt + i]);
                    kg[i] = elem(kp, 4 * kt + i) * fast_exp2(gl[i] - G[4 * kt + i]);
                }
                kgF[kt] = pack4(kg[0], kg[1], kg[2], kg[3]);
                if (r == 0)
                    __builtin_nontemporal_store(
                        f32x4{fast_exp2(gl[0]), fast_exp2(gl[1]), fast_exp2(gl[2]), fast_exp2(gl[3])},
                        reinterpret_cast<f32x4*>(brec + BREC_DECAY + kt * 64 + q4 * 16));
            }
        });
#pragma unroll
        for (int j = 0; j < 4; ++j)
            __builtin_nontemporal_store(
                u32x4{kgF[2 * j].x, kgF[2 * j].y, kgF[2 * j + 1].x, kgF[2 * j + 1].y},
                reinterpret_cast<u32x4*>(brec + BREC_KG + j * 1024 + lane * 16));
    }

    // ---- u = A @ bf16(v * beta) (kernels.py:173-174) ----------------------
    // One 16x16x16 tile per 16 value columns; u lands as
    // u[4*q4 + i][16*vt + r], the order stage 2 subtracts it in.  The
    // transposes below go through the matrix core (tile_T).  In the fused
    // forward's slot the operands go in u's place instead (FREC_*).
    if constexpr (U_IN_SLOT) {
#pragma unroll
        for (int vt = 0; vt < 8; ++vt)
            *reinterpret_cast<u32x2*>(rec + REC_U + vt * 512 + lane * 8) = vp.v[vt];
        *reinterpret_cast<u32x2*>(rec + FREC_A + lane * 8) = ainv_bf;
        if (q4 == 0) *reinterpret_cast<float*>(rec + FREC_BETA + 4 * r) = beta;
    } else {
#pragma unroll
        for (int vt = 0; vt < 8; ++vt) {
            const u32x2 ub = form_u(vp.v[vt], beta, A_op, eye);
            *reinterpret_cast<u32x2*>(rec + REC_U + vt * 512 + lane * 8) = ub;
            if (p.dbg_u) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int row = 4 * q4 + i;
                    if (row < nvalid) {
                        const int64_t o = ((sp.tok0 + t0 + row) * HV + hv) * DK + 16 * vt + r;
                        p.dbg_u[o] = (uint16_t)(i == 0 ? ub.x : i == 1 ? (ub.x >> 16)
                                                : i == 2 ? ub.y : (ub.y >> 16));
                    }
                }
            }
        }
    }

    // ---- w = A @ bf16(bf16(k^ * beta) * 2^G) (kernels.py:171-172), and
    // qg = bf16(q^ * 2^G), the gated query stage 2 multiplies the state by
    // (kernels.py:269).  w is computed transposed, w^T = kb^T @ A^T, so that
    // tile kt lands as w[r][16*kt + 4*q4 + i]: F order, stage 2's operand.
    u32x2 qgp[8], kbF[8];
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
        float kb[4], qg[4], e[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            e[i] = fast_exp2(G[4 * kt + i]);
            kb[i] = round_bf(elem(kp, 4 * kt + i) * beta) * e[i];
            qg[i] = elem(qp, 4 * kt + i) * e[i];
        }
        kbF[kt] = pack4(kb[0], kb[1], kb[2], kb[3]);
        qgp[kt] = pack4(qg[0], qg[1], qg[2], qg[3]);
        // the state's decay 2^G_last (kernels.py:282-290): on the chunk's
        // last row, 2^G is it
        if (r == last)
            *reinterpret_cast<f32x4*>(rec + REC_DECAY + kt * 64 + q4 * 16) = f32x4{e[0], e[1], e[2], e[3]};
    }
    // (the backward's recompute produces no o and never reads qg)
    if constexpr (K1M != K1_BOTH) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const u32x4 qgj = {qgp[2 * j].x, qgp[2 * j].y, qgp[2 * j + 1].x, qgp[2 * j + 1].y};
            *reinterpret_cast<u32x4*>(rec + REC_QG + j * 1024 + lane * 16) = qgj;
        }
    }
    // The record holds -w (stage 2 forms u - w @ hc^T as one accumulation
    // that starts at u): the product with -A, exact since negation commutes
    // with the bf16 products, the fp32 sums and the rounding.
    u32x2 wpk[8];
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
        const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
        wpk[kt] = pack4(mfma_bf16_16x16x16(tile_T(kbF[kt], eye), A_neg, zero));
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const u32x4 wj = {wpk[2 * j].x, wpk[2 * j].y, wpk[2 * j + 1].x, wpk[2 * j + 1].y};
        *reinterpret_cast<u32x4*>(rec + REC_W + j * 1024 + lane * 16) = wj;
    }

    // ---- kg = bf16(k^ * 2^(G_last - G)) (kernels.py:282-290), stored in T
    // order (stage 2's A operand).
    bcast_last([&](auto from_last) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            u32x2 kgT[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int kt = 2 * j + h;
                float kg[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    kg[i] = elem(kp, 4 * kt + i) * fast_exp2(from_last(G[4 * kt + i]) - G[4 * kt + i]);
                kgT[h] = __builtin_bit_cast(u32x2, tile_T(pack4(kg[0], kg[1], kg[2], kg[3]), eye));
            }
            *reinterpret_cast<u32x4*>(rec + REC_KG + j * 1024 + lane * 16) =
                u32x4{kgT[0].x, kgT[0].y, kgT[1].x, kgT[1].y};
        }
    });

    // ---- optional reference-layout intermediates (kernels.py:125,153,178-184)
    if (p.dbg_w && valid) {
        const int64_t bt16 = (tok * HV + hv) * BT + 4 * q4;
        *reinterpret_cast<u32x2*>(p.dbg_Aqk + bt16) = aqk_bf;
        *reinterpret_cast<u32x2*>(p.dbg_A_inv + bt16) = ainv_bf;
#pragma unroll
        for (int kt = 0; kt < 8; ++kt) {
            *reinterpret_cast<u32x2*>(p.dbg_w + vrowoff + 16 * kt + colbase) = wpk[kt] ^ 0x80008000u;
            *reinterpret_cast<f32x4*>(p.dbg_g + vrowoff + 16 * kt + colbase) =
                f32x4{G[4 * kt + 0], G[4 * kt + 1], G[4 * kt + 2], G[4 * kt + 3]};
        }
    }
}

// One chunk (value head hv, chunk c of sequence sp).  FULL: all 16 rows
// are tokens (every chunk but a sequence's partial last one), so the
// row-validity selects and the rows mid = 8, last = 15 are compile-time.
// GB16: g is bf16 (else fp32).
template <int K1M, bool FULL, bool GB16>
__device__ __forceinline__ void k1_chunk(const Params& p, int hv, int c, const SeqSpan& sp,
                                         float* sL, float* sX, uint8_t* rec) {
    K1In<GB16, K1M == K1_BOTH> in;
    k1_load<K1M, FULL, GB16>(p, hv, c, sp, in);
    const float* biasp = k1_bias(p, hv);
    const float ea = k1_ea(p, hv);
    k1_compute<K1M, FULL, GB16>(p, hv, c, sp, in, biasp, ea, sL, sX, rec);
}

}  // namespace
}  // namespace kda
