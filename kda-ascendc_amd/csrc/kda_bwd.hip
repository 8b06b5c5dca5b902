// Backward of the KDA BT=16 chunked forward on gfx950.
//
// The reference is forward-only (/root/reference/README.md:420); its
// analysis of the training graph (/root/reference/docs/KDA_ANALYSIS.md:134-165,
// FLA's chunk_kda_bwd) is: recompute w/u and the chunk states, then the
// reverse recurrence of the state gradient, then the per-chunk WY, gram,
// gate and l2norm gradients and the reverse cumsum of dg.  Here, after the
// recompute (stage 1, then stage 2 storing bf16 h and v_new per chunk, then
// stage 1 again writing the backward records):
//
//   bwd_state_kernel  one wave per (sequence, value head, 16 value
//                     columns), chunks in reverse order, the state gradient
//                     dh [K, 16] resident in eight 16x16 fp32 accumulator
//                     tiles (the forward stage 2's layout):
//                       dv_new = Aqk^T dO + kg dh'
//                       dh     = 2^G_last * dh' + (scale qg)^T dO - w^T dv_new
//                     storing bf16 dh' (the gradient of the state after the
//                     chunk) and dv_new per chunk, and dh0.
//   bwd_chunk_kernel  one work-group per (sequence, q/k head, chunk), all
//                     chunks in parallel, looping over the value heads of a
//                     q/k head: the three products over V on the matrix
//                     cores (dqg = scale dO h^T, dw = -dv_new h^T,
//                     dkg = v_new dh'^T), then the intra-chunk gradients
//                     in fp32 (solve, grams, recentred gates, beta, the
//                     gate and the l2norm), dq / dk summed over the group.
//   gate_reduce       dA_log and ddt_bias from per-chunk partial sums, in
//                     a fixed order (deterministic).
//
// Notation: chunk rows i < n valid; h = S^T [K, V]; E = 2^G; qg = q^ E,
// kg = k^ 2^(G_l - G), kb = beta k^ E, vb = beta v, A = (I + L)^-1,
// L = beta_i tril_strict(kp km^T), Aqk = scale tril(qp km^T) with the
// recentred kp = k^ 2^(G - G_m), qp = q^ 2^(G - G_m), km = k^ 2^(G_m - G).
#include "kda_common.h"

namespace kda {

namespace {

constexpr float LN2 = 0.6931471805599453f;

// ---------------------------------------------------------------------------
// Reverse state chain.
// ---------------------------------------------------------------------------

// The operands of one chunk step (backward record, kda_common.h, and dO).
struct BwdOps {
    u32x4 kg[4];
    u32x4 upd[8];
    u32x2 aqkT;
    f32x4 dec[8];
    u32x2 dop;  // dO[4*q4 + i][16*vt + x] as the 16x16x16 B operand
};

__device__ __forceinline__ void load_bwd_ops(const uint8_t* rec, const uint16_t* drow, bool dvalid,
                                             int lane, int q4, BwdOps& op) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
        op.kg[j] = *reinterpret_cast<const u32x4*>(rec + BREC_KG + j * 1024 + lane * 16);
#pragma unroll
    for (int kt = 0; kt < 8; ++kt)
        op.upd[kt] = *reinterpret_cast<const u32x4*>(rec + BREC_UPD + kt * 1024 + lane * 16);
    op.aqkT = *reinterpret_cast<const u32x2*>(rec + BREC_AQKT + lane * 8);
#pragma unroll
    for (int kt = 0; kt < 8; ++kt)
        op.dec[kt] = *reinterpret_cast<const f32x4*>(rec + BREC_DECAY + kt * 64 + q4 * 16);
    op.dop = u32x2{0u, 0u};
    if (dvalid) op.dop = *reinterpret_cast<const u32x2*>(drow);
}

// Fp32 [K, V] tile slice of lane (x, q4), v = 16*vt + x: D[kt][i] = M[16*kt + 4*q4 + i][v]
// for a state stored [V, K] (v_first) or [K, V].
__device__ __forceinline__ void load_state_T(const float* src, bool v_first, int v, int q4,
                                             f32x4 (&D)[8]) {
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
        D[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (src) {
            const int k0 = 16 * kt + 4 * q4;
            if (v_first) {
                D[kt] = *reinterpret_cast<const f32x4*>(src + (int64_t)v * DK + k0);
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) D[kt][i] = src[(int64_t)(k0 + i) * DK + v];
            }
        }
    }
}

__device__ __forceinline__ void store_state_T(float* dst, bool v_first, int v, int q4,
                                              const f32x4 (&D)[8]) {
    if (!dst) return;
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
        const int k0 = 16 * kt + 4 * q4;
        if (v_first) {
            *reinterpret_cast<f32x4*>(dst + (int64_t)v * DK + k0) = D[kt];
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) dst[(int64_t)(k0 + i) * DK + v] = D[kt][i];
        }
    }
}

__global__ __launch_bounds__(64) void bwd_state_kernel(Params p) {
    const int lane = threadIdx.x;
    const int x = lane & 15, q4 = lane >> 4, j4 = lane & 3;
    const int nbh = (p.cu_seqlens ? p.N : p.B) * p.HV;
    // XCD-aware as stage 2: the 8 value tiles of a head share one L2.
    const int wg = blockIdx.x;
    const int lin = (wg & 7) * nbh + (wg >> 3);
    const int bh = lin >> 3;
    const int vt = lin & 7;
    const int hv = bh - (bh / p.HV) * p.HV;
    const SeqSpan sp = seq_span(p, bh);
    const int v = 16 * vt + x;
    const int64_t sbase = (int64_t)bh * DK * DK;
    const bool v_first = p.h0_v_first != 0;

    f32x4 D[8];
    load_state_T(p.dht ? p.dht + sbase : nullptr, v_first, v, q4, D);
    if (sp.nt > 0) {
        const int col = 16 * vt + 4 * (x >> 2);
        const uint8_t* recs = p.ws + sp.rec0 * REC_BYTES;
        uint16_t* dh_out = p.tr_dh + sp.rec0 * TR_H_ELEMS + col;
        uint16_t* dvn_out = p.tr_dvn + sp.rec0 * TR_VN_ELEMS + col;
        // this lane's dO row piece: token 16*c + 4*q4 + j4, columns col..col+3
        const int64_t dstride = (int64_t)p.HV * DK;
        const uint16_t* dbase = p.dout + (sp.tok0 * p.HV + hv) * DK + col;
        auto drow = [&](int c) { return dbase + (int64_t)(c * BT + 4 * q4 + j4) * dstride; };
        auto dval = [&](int c) { return c * BT + 4 * q4 + j4 < sp.len; };

        BwdOps cur, nxt;
        int c = sp.nt - 1;
        load_bwd_ops(recs + (int64_t)c * REC_BYTES, drow(c), dval(c), lane, q4, cur);
        for (; c >= 0; --c) {
            if (c > 0)
                load_bwd_ops(recs + (int64_t)(c - 1) * REC_BYTES, drow(c - 1), dval(c - 1), lane,
                             q4, nxt);
            // dh' = the gradient of the state after chunk c, as bf16 B operands
            u32x4 hb[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                hb[j] = u32x4{pack2(D[2 * j][0], D[2 * j][1]), pack2(D[2 * j][2], D[2 * j][3]),
                              pack2(D[2 * j + 1][0], D[2 * j + 1][1]),
                              pack2(D[2 * j + 1][2], D[2 * j + 1][3])};
            const u32x2 dt = quad_transpose(cur.dop.x, cur.dop.y, j4);
            const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
            f32x4 dvn = mfma_bf16_16x16x16(as_i16x4(cur.aqkT), as_i16x4(dt), zero);
#pragma unroll
            for (int j = 0; j < 4; ++j) dvn = mfma_bf16_16x16x32(as_bf16x8(cur.kg[j]), as_bf16x8(hb[j]), dvn);
            // store dh' row pieces (after the products have their operands)
            uint16_t* dhc = dh_out + (int64_t)c * TR_H_ELEMS;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const u32x2 t0 = quad_transpose(hb[j].x, hb[j].y, j4);
                const u32x2 t1 = quad_transpose(hb[j].z, hb[j].w, j4);
                const int k0 = 32 * j + 4 * q4 + j4;
                *reinterpret_cast<u32x2*>(dhc + (int64_t)k0 * DK) = t0;
                *reinterpret_cast<u32x2*>(dhc + (int64_t)(k0 + 16) * DK) = t1;
            }
            const u32x2 dvb = {pack2(dvn[0], dvn[1]), pack2(dvn[2], dvn[3])};
            const u32x2 dvt = quad_transpose(dvb.x, dvb.y, j4);
            *reinterpret_cast<u32x2*>(dvn_out + (int64_t)c * TR_VN_ELEMS + (4 * q4 + j4) * DK) = dvt;
            // dh = 2^G_last * dh' + [scale qg | -w]^T [dO ; dv_new]
            const u32x4 bop = {dt.x, dt.y, dvb.x, dvb.y};
#pragma unroll
            for (int kt = 0; kt < 8; ++kt) {
                D[kt] = D[kt] * cur.dec[kt];
                D[kt] = mfma_bf16_16x16x32(as_bf16x8(cur.upd[kt]), as_bf16x8(bop), D[kt]);
            }
            if (c > 0) cur = nxt;
        }
    }
    store_state_T(p.dh0 ? p.dh0 + sbase : nullptr, v_first, v, q4, D);
}

// ---------------------------------------------------------------------------
// Per-chunk gradients.
// ---------------------------------------------------------------------------

constexpr int CT = 256;    // threads: row i = t / 16 owns columns 8*(t % 16) .. +7
constexpr int LD = DK + 4; // fp32 row stride of the [16][128] LDS matrices

struct ChunkSmem {
    float kp[BT][LD], km[BT][LD], qp[BT][LD], kb[BT][LD], vb[BT][LD];
    float dw[BT][LD], dvn[BT][LD], dqg[BT][LD], dkg[BT][LD], gsc[BT][LD];
    float el[DK], del[DK];
    float lraw[BT][BT + 1], ainv[BT][BT + 1], da[BT][BT + 1], m1[BT][BT + 1];
    float dlr[BT][BT + 1], daqm[BT][BT + 1];
    float red[CT / 64];
};

__device__ __forceinline__ void load8(const uint16_t* src, bool valid, float (&out)[8]) {
    u32x4 w = {0u, 0u, 0u, 0u};
    if (valid) w = *reinterpret_cast<const u32x4*>(src);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        out[2 * j] = __builtin_bit_cast(float, w[j] << 16);
        out[2 * j + 1] = __builtin_bit_cast(float, w[j] & 0xffff0000u);
    }
}

__device__ __forceinline__ void store8(uint16_t* dst, const float (&x)[8]) {
    *reinterpret_cast<u32x4*>(dst) =
        u32x4{pack2(x[0], x[1]), pack2(x[2], x[3]), pack2(x[4], x[5]), pack2(x[6], x[7])};
}

// Sum over the 16 threads of a row (lanes 16*m .. 16*m + 15 of a wave).
__device__ __forceinline__ float row_sum16(float s) {
    s += __shfl_xor(s, 1);
    s += __shfl_xor(s, 2);
    s += __shfl_xor(s, 4);
    s += __shfl_xor(s, 8);
    return s;
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.f / (1.f + expf(-x)); }

__global__ __launch_bounds__(CT) void bwd_chunk_kernel(Params p) {
    __shared__ ChunkSmem sm;
    const int t = threadIdx.x;
    const int lane = t & 63, w = t >> 6;
    const int i = t >> 4;          // row (and row of the 16x16 mapping)
    const int cb = t & 15;         // column of the 16x16 mapping
    const int c0 = 8 * cb;         // first of this thread's 8 columns
    const int H = p.H, HV = p.HV, rep = HV / H;
    const bool gate_grads = p.use_gate && p.tr_part;

    int h, c, seq;  // q/k head, chunk, batch row or sequence
    if (p.cu_seqlens) {
        h = blockIdx.x / p.NS;
        const int xs = blockIdx.x - h * p.NS;
        seq = find_sequence(p, xs, lane);
        const SeqSpan s0 = seq_span(p, seq * HV);
        c = (int)((int64_t)xs - s0.rec0);  // rec0 of value head 0 is bos/16 + n
        if (c < 0 || c >= s0.nt) {
            // a gap slot: its partial sums are zero
            if (gate_grads && t <= DK) {
                for (int gi = 0; gi < rep; ++gi)
                    p.tr_part[((int64_t)(h * rep + gi) * p.NS + xs) * PART_STRIDE + t] = 0.f;
            }
            return;
        }
    } else {
        c = blockIdx.x % p.NT;
        const int bq = blockIdx.x / p.NT;
        seq = bq / H;
        h = bq - seq * H;
    }
    const SeqSpan sq = seq_span(p, seq * HV + h * rep);
    const int nvalid = min(BT, sq.len - c * BT);
    const int mid = min(BT / 2, nvalid - 1), last = nvalid - 1;
    const bool valid = i < nvalid;
    const int64_t tok = sq.tok0 + c * BT + i;

    // ---- q^, k^ (kernels.py:108-113), once per q/k head ------------------
    float qv[8], kv[8], qn[8], kn[8];
    load8(p.q + (tok * H + h) * DK + c0, valid, qv);
    load8(p.k + (tok * H + h) * DK + c0, valid, kv);
    float rq = 1.f, rk = 1.f;
    if (p.use_l2norm) {
        float sq2 = 0.f, sk2 = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            sq2 = fmaf(qv[j], qv[j], sq2);
            sk2 = fmaf(kv[j], kv[j], sk2);
        }
        sq2 = row_sum16(sq2);
        sk2 = row_sum16(sk2);
        rq = 1.f / sqrtf(sq2 + L2_EPS);
        rk = 1.f / sqrtf(sk2 + L2_EPS);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        qn[j] = p.use_l2norm ? round_bf(qv[j] * rq) : qv[j];
        kn[j] = p.use_l2norm ? round_bf(kv[j] * rk) : kv[j];
    }
    float dQN[8], dKN[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) dQN[j] = dKN[j] = 0.f;

    for (int gi = 0; gi < rep; ++gi) {
        const int hv = h * rep + gi;
        const SeqSpan sp = seq_span(p, seq * HV + hv);
        const int64_t rec = sp.rec0 + c;
        const int64_t vrow = (tok * HV + hv) * DK;  // v/g/dO element offset of row i

        // ---- phase 1: gates, cumsum, recentred operands ------------------
        float vv[8], gr[8], dvn[8];
        load8(p.v + vrow + c0, valid, vv);
        load8(p.tr_dvn + rec * TR_VN_ELEMS + i * DK + c0, valid, dvn);
        if (p.g_bf16) {
            load8(static_cast<const uint16_t*>(p.g) + vrow + c0, valid, gr);
        } else {
            const float* gs = static_cast<const float*>(p.g) + vrow + c0;
#pragma unroll
            for (int j = 0; j < 8; ++j) gr[j] = valid ? gs[j] : 0.f;
        }
        float beta = 0.f;
        if (valid) {
            const int64_t bi = tok * HV + hv;
            beta = p.beta_bf16 ? bf2f(static_cast<const uint16_t*>(p.beta)[bi])
                               : static_cast<const float*>(p.beta)[bi];
        }
        const float braw = beta;
        if (p.use_beta_sigmoid) beta = valid ? sigmoidf_(braw) : 0.f;
        const float ea = p.use_gate ? expf(p.A_log[hv]) : 0.f;
        float bias[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            bias[j] = (p.use_gate && p.dt_bias) ? p.dt_bias[hv * DK + c0 + j] : 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float gv;
            if (p.use_gate) gv = p.lower_bound * sigmoidf_(ea * (gr[j] + bias[j]));
            else gv = gr[j];
            sm.gsc[i][c0 + j] = valid ? gv : 0.f;
            sm.dvn[i][c0 + j] = dvn[j];
        }
        __syncthreads();
        if ((p.use_gate || p.g_log) && t < DK) {
            float run = 0.f;
#pragma unroll
            for (int r = 0; r < BT; ++r) {
                run += sm.gsc[r][t];
                sm.gsc[r][t] = run * RCP_LN2;
            }
        }
        __syncthreads();
        if (t < DK) sm.el[t] = exp2f(sm.gsc[last][t]);
        float E[8], eq[8], ek[8], kgl[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float G = sm.gsc[i][c0 + j];
            const float Gm = sm.gsc[mid][c0 + j];
            const float Gl = sm.gsc[last][c0 + j];
            E[j] = valid ? exp2f(G) : 0.f;
            eq[j] = valid ? exp2f(G - Gm) : 0.f;
            ek[j] = valid ? exp2f(Gm - G) : 0.f;
            kgl[j] = valid ? exp2f(Gl - G) : 0.f;
            sm.qp[i][c0 + j] = qn[j] * eq[j];
            sm.kp[i][c0 + j] = kn[j] * eq[j];
            sm.km[i][c0 + j] = kn[j] * ek[j];
            sm.kb[i][c0 + j] = round_bf(round_bf(kn[j] * beta) * E[j]);
            sm.vb[i][c0 + j] = round_bf(vv[j] * beta);
        }

        // ---- phase 2: products over V on the matrix cores ----------------
        // Wave w owns k-tiles 2w, 2w+1.  Lane (x, q4) feeds row x of dO /
        // dv_new / v_new and row 16*kt + x of h / dh', v columns
        // 32*jv + 8*q4 .. +7, as 16x16x32 operands.
        {
            const int x = lane & 15, q4 = lane >> 4;
            const bool xv = x < nvalid;
            const uint16_t* hrec = p.tr_h + rec * TR_H_ELEMS;
            const uint16_t* dhrec = p.tr_dh + rec * TR_H_ELEMS;
            const uint16_t* vnrec = p.tr_vn + rec * TR_VN_ELEMS + x * DK + 8 * q4;
            const uint16_t* dvrec = p.tr_dvn + rec * TR_VN_ELEMS + x * DK + 8 * q4;
            const uint16_t* dorow = p.dout + ((sq.tok0 + c * BT + x) * HV + hv) * DK + 8 * q4;
            f32x4 aq[2], aw[2], ak[2], adq = {0.f, 0.f, 0.f, 0.f};
            float pel[2] = {0.f, 0.f};
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) aq[tt] = aw[tt] = ak[tt] = adq;
#pragma unroll
            for (int jv = 0; jv < 4; ++jv) {
                u32x4 a_do = {0u, 0u, 0u, 0u}, a_dv = {0u, 0u, 0u, 0u}, a_vn = {0u, 0u, 0u, 0u};
                if (xv) {
                    a_do = *reinterpret_cast<const u32x4*>(dorow + 32 * jv);
                    a_dv = *reinterpret_cast<const u32x4*>(dvrec + 32 * jv);
                    a_vn = *reinterpret_cast<const u32x4*>(vnrec + 32 * jv);
                }
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
                    const int kt = 2 * w + tt;
                    const int64_t off = (int64_t)(16 * kt + x) * DK + 32 * jv + 8 * q4;
                    const u32x4 bh = *reinterpret_cast<const u32x4*>(hrec + off);
                    const u32x4 bd = *reinterpret_cast<const u32x4*>(dhrec + off);
                    aq[tt] = mfma_bf16_16x16x32(as_bf16x8(a_do), as_bf16x8(bh), aq[tt]);
                    aw[tt] = mfma_bf16_16x16x32(as_bf16x8(a_dv), as_bf16x8(bh), aw[tt]);
                    ak[tt] = mfma_bf16_16x16x32(as_bf16x8(a_vn), as_bf16x8(bd), ak[tt]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        pel[tt] = fmaf(__builtin_bit_cast(float, bh[e] << 16),
                                       __builtin_bit_cast(float, bd[e] << 16), pel[tt]);
                        pel[tt] = fmaf(__builtin_bit_cast(float, bh[e] & 0xffff0000u),
                                       __builtin_bit_cast(float, bd[e] & 0xffff0000u), pel[tt]);
                    }
                }
                if (w == 0) adq = mfma_bf16_16x16x32(as_bf16x8(a_do), as_bf16x8(a_vn), adq);
            }
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                const int kt = 2 * w + tt;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int row = 4 * q4 + e;
                    sm.dqg[row][16 * kt + x] = p.scale * aq[tt][e];
                    sm.dw[row][16 * kt + x] = -aw[tt][e];
                    sm.dkg[row][16 * kt + x] = ak[tt][e];
                }
                float s = pel[tt];
                s += __shfl_xor(s, 16);
                s += __shfl_xor(s, 32);
                if (q4 == 0) sm.del[16 * kt + x] = s;
            }
            if (w == 0) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int row = 4 * q4 + e;
                    sm.daqm[row][x] = row >= x ? p.scale * adq[e] : 0.f;
                }
            }
        }
        __syncthreads();

        // ---- phase 3: L = beta tril_strict(kp km^T), A = (I + L)^-1 -------
        {
            float s = 0.f;
            for (int k = 0; k < DK; k += 4) {
                const f32x4 a = *reinterpret_cast<const f32x4*>(&sm.kp[i][k]);
                const f32x4 b = *reinterpret_cast<const f32x4*>(&sm.km[cb][k]);
                s = fmaf(a[0], b[0], s);
                s = fmaf(a[1], b[1], s);
                s = fmaf(a[2], b[2], s);
                s = fmaf(a[3], b[3], s);
            }
            sm.lraw[i][cb] = s;
            sm.m1[i][cb] = (i > cb) ? beta * s : 0.f;  // L, read by the solve
        }
        __syncthreads();
        if (t < BT) {
            // column s = t of A_inv: a[s] = 1, a[r > s] = -sum_{j<r} L[r][j] a[j]
            float a[BT];
#pragma unroll
            for (int r = 0; r < BT; ++r) {
                float acc = 0.f;
#pragma unroll
                for (int jj = 0; jj < r; ++jj) acc = fmaf(-sm.m1[r][jj], a[jj], acc);
                a[r] = (r > t) ? acc : (r == t ? 1.f : 0.f);
            }
#pragma unroll
            for (int r = 0; r < BT; ++r) sm.ainv[r][t] = a[r];
        }
        __syncthreads();

        // ---- phase 4: dA = dw kb^T + du vb^T; dkb = A^T dw, dvb = A^T du --
        {
            float s = 0.f;
            for (int k = 0; k < DK; k += 4) {
                const f32x4 a = *reinterpret_cast<const f32x4*>(&sm.dw[i][k]);
                const f32x4 b = *reinterpret_cast<const f32x4*>(&sm.kb[cb][k]);
                const f32x4 a2 = *reinterpret_cast<const f32x4*>(&sm.dvn[i][k]);
                const f32x4 b2 = *reinterpret_cast<const f32x4*>(&sm.vb[cb][k]);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    s = fmaf(a[e], b[e], s);
                    s = fmaf(a2[e], b2[e], s);
                }
            }
            sm.da[i][cb] = s;
        }
        float dkb[8], dvb[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) dkb[j] = dvb[j] = 0.f;
        for (int r = i; r < BT; ++r) {
            const float a = round_bf(sm.ainv[r][i]);  // the bf16 A of w, u (kernels.py:170)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                dkb[j] = fmaf(a, sm.dw[r][c0 + j], dkb[j]);
                dvb[j] = fmaf(a, sm.dvn[r][c0 + j], dvb[j]);
            }
        }
        __syncthreads();

        // ---- phase 5: dL = -A^T dA A^T (strictly lower), dLr = beta dL ----
        {
            float s = 0.f;
#pragma unroll
            for (int m = 0; m < BT; ++m) s = fmaf(sm.da[i][m], sm.ainv[cb][m], s);
            sm.m1[i][cb] = s;  // (dA A^T)[i][cb]
        }
        __syncthreads();
        float dbl;
        {
            float s = 0.f;
#pragma unroll
            for (int m = 0; m < BT; ++m) s = fmaf(sm.ainv[m][i], sm.m1[m][cb], s);
            const float dl = (i > cb) ? -s : 0.f;
            sm.dlr[i][cb] = beta * dl;
            dbl = row_sum16(dl * sm.lraw[i][cb]);
        }
        __syncthreads();

        // ---- phase 6: the row-wise gradients ------------------------------
        float dkp[8], dqp[8], dkm[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) dkp[j] = dqp[j] = dkm[j] = 0.f;
#pragma unroll 4
        for (int b = 0; b < BT; ++b) {
            const float l1 = sm.dlr[i][b], a1 = sm.daqm[i][b];
            const float l2 = sm.dlr[b][i], a2 = sm.daqm[b][i];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float kmv = sm.km[b][c0 + j];
                dkp[j] = fmaf(l1, kmv, dkp[j]);
                dqp[j] = fmaf(a1, kmv, dqp[j]);
                dkm[j] = fmaf(l2, sm.kp[b][c0 + j], dkm[j]);
                dkm[j] = fmaf(a2, sm.qp[b][c0 + j], dkm[j]);
            }
        }
        float dbeta = 0.f, dv[8], dG[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float dqg = sm.dqg[i][c0 + j];
            const float dkg = sm.dkg[i][c0 + j];
            const float qp = qn[j] * eq[j], kp = kn[j] * eq[j], km = kn[j] * ek[j];
            const float qg = qn[j] * E[j], kg = kn[j] * kgl[j];
            const float kb = sm.kb[i][c0 + j];
            dQN[j] += dqg * E[j] + dqp[j] * eq[j];
            dKN[j] += dkb[j] * beta * E[j] + dkg * kgl[j] + dkp[j] * eq[j] + dkm[j] * ek[j];
            dbeta = fmaf(dkb[j], kn[j] * E[j], dbeta);
            dbeta = fmaf(dvb[j], vv[j], dbeta);
            dv[j] = dvb[j] * beta;
            dG[j] = LN2 * (dkb[j] * kb + dqg * qg - dkg * kg + dqp[j] * qp + dkp[j] * kp -
                           dkm[j] * km);
        }
        dbeta = row_sum16(dbeta) + dbl;
        if (valid) {
            store8(p.dv + vrow + c0, dv);
            if (cb == 0) {
                const float db = p.use_beta_sigmoid ? dbeta * beta * (1.f - beta) : dbeta;
                const int64_t bi = tok * HV + hv;
                if (p.beta_bf16) static_cast<uint16_t*>(p.dbeta)[bi] = f2bf(db);
                else static_cast<float*>(p.dbeta)[bi] = db;
            }
        }
        __syncthreads();  // every read of gsc, dkg and the 16x16 scratch is done
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            sm.gsc[i][c0 + j] = valid ? dG[j] : 0.f;
            sm.dkg[i][c0 + j] = valid ? sm.dkg[i][c0 + j] * kn[j] * kgl[j] : 0.f;
        }
        __syncthreads();

        // ---- phase 7: per column, the last row's dG, the reverse cumsum of
        // dG into dgate, and the gate (kernels.py:115-124) ------------------
        if (t < DK) {
            const int k = t;
            float s = 0.f;
#pragma unroll
            for (int r = 0; r < BT; ++r) s += sm.dkg[r][k];
            sm.gsc[last][k] += LN2 * (s + sm.el[k] * sm.del[k]);
            const float bk = (p.use_gate && p.dt_bias) ? p.dt_bias[hv * DK + k] : 0.f;
            float run = 0.f, pdt = 0.f, pal = 0.f;
            for (int r = nvalid - 1; r >= 0; --r) {
                run += sm.gsc[r][k];
                const int64_t gidx = ((sq.tok0 + c * BT + r) * HV + hv) * DK + k;
                float dg;
                if (p.use_gate) {
                    const float graw = p.g_bf16 ? bf2f(static_cast<const uint16_t*>(p.g)[gidx])
                                                : static_cast<const float*>(p.g)[gidx];
                    const float sarg = graw + bk;
                    const float sg = sigmoidf_(ea * sarg);
                    dg = RCP_LN2 * run * p.lower_bound * sg * (1.f - sg) * ea;
                    pdt += dg;
                    pal = fmaf(dg, sarg, pal);
                } else if (p.g_log) {
                    dg = RCP_LN2 * run;
                } else {
                    dg = sm.gsc[r][k];
                }
                if (p.g_bf16) static_cast<uint16_t*>(p.dg)[gidx] = f2bf(dg);
                else static_cast<float*>(p.dg)[gidx] = dg;
            }
            if (gate_grads) {
                p.tr_part[rec * PART_STRIDE + k] = pdt;
                float a = pal;
                a += __shfl_xor(a, 1);
                a += __shfl_xor(a, 2);
                a += __shfl_xor(a, 4);
                a += __shfl_xor(a, 8);
                a += __shfl_xor(a, 16);
                a += __shfl_xor(a, 32);
                if (lane == 0) sm.red[w] = a;
            }
        }
        __syncthreads();
        if (gate_grads && t == 0) p.tr_part[rec * PART_STRIDE + DK] = sm.red[0] + sm.red[1];
    }

    // ---- l2norm backward, dq / dk summed over the group -------------------
    if (p.use_l2norm) {
        float dq_dot = 0.f, dk_dot = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            dq_dot = fmaf(qv[j] * rq, dQN[j], dq_dot);
            dk_dot = fmaf(kv[j] * rk, dKN[j], dk_dot);
        }
        dq_dot = row_sum16(dq_dot);
        dk_dot = row_sum16(dk_dot);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            dQN[j] = rq * (dQN[j] - qv[j] * rq * dq_dot);
            dKN[j] = rk * (dKN[j] - kv[j] * rk * dk_dot);
        }
    }
    if (valid) {
        store8(p.dq + (tok * H + h) * DK + c0, dQN);
        store8(p.dk + (tok * H + h) * DK + c0, dKN);
    }
}

// dA_log[hv] and ddt_bias[hv, :] summed over the chunk partials of value
// head hv, in record order.
__global__ __launch_bounds__(DK) void gate_reduce_kernel(Params p) {
    const int hv = blockIdx.x, t = threadIdx.x;
    float acc = 0.f, accA = 0.f;
    if (p.cu_seqlens) {
        const float* base = p.tr_part + (int64_t)hv * p.NS * PART_STRIDE;
        for (int x = 0; x < p.NS; ++x) {
            acc += base[(int64_t)x * PART_STRIDE + t];
            if (t == 0) accA += base[(int64_t)x * PART_STRIDE + DK];
        }
    } else {
        for (int b = 0; b < p.B; ++b) {
            const float* base = p.tr_part + (int64_t)(b * p.HV + hv) * p.NT * PART_STRIDE;
            for (int c = 0; c < p.NT; ++c) {
                acc += base[(int64_t)c * PART_STRIDE + t];
                if (t == 0) accA += base[(int64_t)c * PART_STRIDE + DK];
            }
        }
    }
    if (p.ddt_bias) p.ddt_bias[hv * DK + t] = acc;
    if (p.dA_log && t == 0) p.dA_log[hv] = accA;
}

}  // namespace

hipError_t launch_bwd_state(const Params& p, hipStream_t stream) {
    const int64_t grid = (int64_t)(p.cu_seqlens ? p.N : p.B) * p.HV * 8;
    hipLaunchKernelGGL(bwd_state_kernel, dim3((unsigned)grid), dim3(64), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_bwd_chunk(const Params& p, hipStream_t stream) {
    const int64_t grid = p.cu_seqlens ? (int64_t)p.H * p.NS : (int64_t)p.B * p.H * p.NT;
    hipLaunchKernelGGL(bwd_chunk_kernel, dim3((unsigned)grid), dim3(CT), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_bwd_gate_reduce(const Params& p, hipStream_t stream) {
    hipLaunchKernelGGL(gate_reduce_kernel, dim3((unsigned)p.HV), dim3(DK), 0, stream, p);
    return hipGetLastError();
}

}  // namespace kda
