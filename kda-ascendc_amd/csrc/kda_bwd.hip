// Backward of the KDA BT=16 chunked forward on gfx950.
//
// The reference is forward-only (/root/reference/README.md:420); its
// analysis of the training graph (/root/reference/docs/KDA_ANALYSIS.md:134-165,
// FLA's chunk_kda_bwd) is: recompute w/u and the chunk states, then the
// reverse recurrence of the state gradient, then the per-chunk WY, gram,
// gate and l2norm gradients and the reverse cumsum of dg.  Here, after the
// recompute (one stage-1 pass writing the forward and the backward records,
// then stage 2 storing bf16 h and v_new per chunk):
//
//   k2_kernel<K2_BWD> (kda_k2.hip) the reverse recurrence of the state
//                     gradient dh, stage 2's four-wave layout run over
//                     the backward records in reverse chunk order:
//                       dv_new = Aqk^T dO + kg dh'
//                       dh     = 2^G_last * dh' + (scale qg)^T dO - w^T dv_new
//                     storing bf16 dh' (the gradient of the state after the
//                     chunk) and dv_new per chunk, and dh0.
//   bwd_chunk_kernel  one work-group per (sequence, q/k head, chunk), all
//                     chunks in parallel, looping over the value heads of a
//                     q/k head: the three products over V on the matrix
//                     cores (dqg = scale dO h^T, dw = -dv_new h^T,
//                     dkg = v_new dh'^T), then the intra-chunk gradients
//                     in fp32 (through A = (I + L)^-1 and the gram, both
//                     read from stage 1's record; the recentred gates,
//                     beta, the gate and the l2norm), dq / dk summed over
//                     the group.
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
// Per-chunk gradients.
// ---------------------------------------------------------------------------

constexpr int CT = 256;    // threads: row i = t / 16 owns columns 8*(t % 16) .. +7
constexpr int LD = DK + 4; // fp32 row stride of the [16][128] LDS matrices

// The four waves split the small products on the fp32 16x16x4 matrix op,
// operands read from these tiles: lane (n, k') of a wave supplies
// A[n][4*s + k'] and B[4*s + k'][n] for slab s, and D[m][n] lands in lane
// n + 16*(m/4) item m%4 (kda_common.h).
// 74 KiB, so that two work-groups share a CU.  Tiles are reused once dead:
// dqg first holds the gate cumsum G, dw / dvn later hold dkb / dvb, kp /
// km / qp / dqg end as dG and the gate's column sums, and the 16x16
// scratch takes dA's partial sums.
constexpr int LDB = DK + 8;  // bf16 row stride of the kb / vb tiles
struct ChunkSmem {
    float kp[BT][LD], km[BT][LD], qp[BT][LD];
    float dw[BT][LD], dvn[BT][LD], dqg[BT][LD], dkg[BT][LD];
    uint16_t kb[BT][LDB], vb[BT][LDB];  // bf16-valued by construction
    float el[DK], del[DK], gm[DK], gl[DK];  // 2^G_last, dE_last, G of rows mid / last
    float lraw[BT][BT + 1], ainv[BT][BT + 1], da[BT][BT + 1], m1[BT][BT + 1];
    float dlr[BT][BT + 1], daqm[BT][BT + 1];
    float red[CT / 64];
};

__device__ __forceinline__ void store8(uint16_t* dst, const float (&x)[8]) {
    *reinterpret_cast<u32x4*>(dst) =
        u32x4{pack2(x[0], x[1]), pack2(x[2], x[3]), pack2(x[4], x[5]), pack2(x[6], x[7])};
}

__device__ __forceinline__ void lds_put8(float* dst, const float (&x)[8]) {
    *reinterpret_cast<f32x4*>(dst) = f32x4{x[0], x[1], x[2], x[3]};
    *reinterpret_cast<f32x4*>(dst + 4) = f32x4{x[4], x[5], x[6], x[7]};
}

__device__ __forceinline__ void lds_put8_bf(uint16_t* dst, const float (&x)[8]) {
    *reinterpret_cast<u32x4*>(dst) =
        u32x4{pack2(x[0], x[1]), pack2(x[2], x[3]), pack2(x[4], x[5]), pack2(x[6], x[7])};
}

__device__ __forceinline__ void lds_get8(const float* src, float (&x)[8]) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(src);
    const f32x4 b = *reinterpret_cast<const f32x4*>(src + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        x[j] = a[j];
        x[4 + j] = b[j];
    }
}

// (row_sum16, kda_common.h: the sum over the 16 threads of a row, lanes
// 16*m .. 16*m + 15 of a wave)

// One value head's row data of this thread (row i, columns c0 .. c0+7):
// g is the gate's argument g + dt_bias with the in-kernel gate, else g.
struct HvRow {
    float v[8], g[8], dvn[8];
    float beta, alog;
};

// The same, as loaded: packed rows and raw bits, converted only where they
// are first used, so that no load waits for another's round trip.
struct HvRaw {
    u32x4 v, dvn, g[2];  // g: bf16 in g[0], or fp32 bits in g[0..1]
    f32x4 bias[2];
    uint32_t beta;       // bf16 in the low half, or fp32 bits
    float alog;
    float lraw, ainv;    // Lraw[i][cb], A_inv[i][cb] as stage 1 formed them
};

__device__ __forceinline__ void unpack8(const u32x4& w, float (&out)[8]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        out[2 * j] = __builtin_bit_cast(float, w[j] << 16);
        out[2 * j + 1] = __builtin_bit_cast(float, w[j] & 0xffff0000u);
    }
}

// One value head's matrix-op operands for the products over V (wave w:
// k-tiles 2w, 2w+1), loaded ahead of the intra-chunk work so that their
// latency overlaps it.
struct HdhOps {
    u32x4 bh[4][2], bd[4][2];      // h, dh' rows 16*kt + x, v 32*jv + 8*q4 .. +7
    u32x4 a_do[4], a_dv[4], a_vn[4];  // dO, dv_new, v_new row x, same v
};

// GROUP: grouped value heads (HV > H), the value heads of a q/k head in a
// loop.  Without it the body runs once, and the compiler keeps nothing live
// across iterations (hoisted addresses and row values would otherwise hold
// registers through the whole body).  FULL: a fixed-length batch with T a
// multiple of 16, so every row of every chunk is a token (no row-validity
// selects).
template <bool GROUP, bool FULL>
__global__ __launch_bounds__(CT) __attribute__((amdgpu_waves_per_eu(GROUP ? 1 : 2))) void bwd_chunk_kernel(Params p) {
    __shared__ ChunkSmem sm;
    const int t = threadIdx.x;
    const int lane = t & 63, w = t >> 6;
    const int x = lane & 15, q4 = lane >> 4;  // matrix-op lane coordinates
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
    const bool valid = FULL || i < nvalid;
    const int64_t tok = sq.tok0 + c * BT + i;

    // Every load of a value head is issued before the first wait.  Rows
    // past the chunk's last token read that token's row (in bounds) and are
    // zeroed where they are used; absent operands read kZeroCols.
    const int64_t tokc = sq.tok0 + c * BT + (valid ? i : nvalid - 1);
    const bool has_bias = p.use_gate && p.dt_bias;
    auto load_hv = [&](int hv, HvRaw& r) {
        const SeqSpan sp = seq_span(p, seq * HV + hv);
        const int64_t rec = sp.rec0 + c;
        const int64_t vrow = (tokc * HV + hv) * DK;
        // (the row loads last: an address formed after a load may take that
        // load's destination registers and wait for it)
        const int64_t bi = tokc * HV + hv;
        if (p.beta_bf16) r.beta = static_cast<const uint16_t*>(p.beta)[bi];
        else r.beta = static_cast<const uint32_t*>(p.beta)[bi];
        r.alog = *(p.use_gate ? p.A_log + hv : kZeroCols);
        const float* laf = reinterpret_cast<const float*>(p.la + rec * p.la_stride);
        r.lraw = laf[LA_LRAW / 4 + (i + 16 * (cb >> 2)) * 4 + (cb & 3)];
        r.ainv = laf[LA_AINV / 4 + (i + 16 * (cb >> 2)) * 4 + (cb & 3)];
        const float* biasp = has_bias ? p.dt_bias + hv * DK : kZeroCols;
        r.bias[0] = *reinterpret_cast<const f32x4*>(biasp + c0);
        r.bias[1] = *reinterpret_cast<const f32x4*>(biasp + c0 + 4);
        r.dvn = *reinterpret_cast<const u32x4*>(p.tr_dvn + rec * TR_VN_ELEMS + (cb >> 1) * TR_VN_TILE +
                                                i * 16 + 8 * (cb & 1));
        r.v = *reinterpret_cast<const u32x4*>(p.v + vrow + c0);
        // bf16: 16 bytes (read twice); fp32: 32 bytes
        const uint32_t* gsrc = p.g_bf16
            ? reinterpret_cast<const uint32_t*>(static_cast<const uint16_t*>(p.g) + vrow + c0)
            : reinterpret_cast<const uint32_t*>(static_cast<const float*>(p.g) + vrow + c0);
        r.g[0] = *reinterpret_cast<const u32x4*>(gsrc);
        r.g[1] = *reinterpret_cast<const u32x4*>(gsrc + (p.g_bf16 ? 0 : 4));
    };
    // g is the gate's argument g + dt_bias with the in-kernel gate; rows
    // past the last token hold v = dv_new = beta = 0 and g = dt_bias.
    auto decode_hv = [&](const HvRaw& r, HvRow& o) {
        float v[8], dv[8], g[8];
        unpack8(r.v, v);
        unpack8(r.dvn, dv);
        if (p.g_bf16) {
            unpack8(r.g[0], g);
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                // (vector elements copied out first: a bit cast of the
                // element itself read element 0 whatever j was)
                const uint32_t lo = r.g[0][j], hi = r.g[1][j];
                g[j] = __builtin_bit_cast(float, lo);
                g[4 + j] = __builtin_bit_cast(float, hi);
            }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            o.v[j] = valid ? v[j] : 0.f;
            o.dvn[j] = valid ? dv[j] : 0.f;
            const float gv = valid ? g[j] : 0.f;
            o.g[j] = has_bias ? gv + r.bias[j >> 2][j & 3] : gv;
        }
        const float b = __builtin_bit_cast(float, p.beta_bf16 ? r.beta << 16 : r.beta);
        o.beta = valid ? b : 0.f;
        o.alog = r.alog;
    };
    auto load_ops = [&](int hv, HdhOps& o) {
        const int64_t rec = seq_span(p, seq * HV + hv).rec0 + c;
        const uint16_t* hrec = p.tr_h + rec * TR_H_ELEMS;
        const uint16_t* dhrec = p.tr_dh + rec * TR_H_ELEMS;
        // blocked layouts: v = 32*jv + 8*q4 + e lies in value tile
        // 2*jv + q4/2 at column 8*(q4%2) + e
        const int64_t vnoff = (q4 >> 1) * TR_VN_TILE + x * 16 + 8 * (q4 & 1);
        const uint16_t* vnrec = p.tr_vn + rec * TR_VN_ELEMS + vnoff;
        const uint16_t* dvrec = p.tr_dvn + rec * TR_VN_ELEMS + vnoff;
        const int xr = x < nvalid ? x : nvalid - 1;
        const uint16_t* dorow = p.dout + ((sq.tok0 + c * BT + xr) * HV + hv) * DK + 8 * q4;
#pragma unroll
        for (int jv = 0; jv < 4; ++jv) {
            o.a_do[jv] = *reinterpret_cast<const u32x4*>(dorow + 32 * jv);
            o.a_dv[jv] = *reinterpret_cast<const u32x4*>(dvrec + 2 * jv * TR_VN_TILE);
            o.a_vn[jv] = *reinterpret_cast<const u32x4*>(vnrec + 2 * jv * TR_VN_TILE);
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                const int kt = 2 * w + tt;
                const int64_t off = (2 * jv + (q4 >> 1)) * TR_H_TILE + (16 * kt + x) * 16 +
                                    8 * (q4 & 1);
                o.bh[jv][tt] = *reinterpret_cast<const u32x4*>(hrec + off);
                o.bd[jv][tt] = *reinterpret_cast<const u32x4*>(dhrec + off);
            }
        }
    };
    // Rows x past the last token of a partial chunk as zero (dO, dv_new,
    // v_new); a full chunk skips this without waiting on the loads.
    auto mask_ops = [&](HdhOps& o) {
        if (nvalid < BT && x >= nvalid) {
#pragma unroll
            for (int jv = 0; jv < 4; ++jv) o.a_do[jv] = o.a_dv[jv] = o.a_vn[jv] = u32x4{0u, 0u, 0u, 0u};
        }
    };

    // ---- q^, k^ (kernels.py:108-113), once per q/k head; the raw rows stay
    // packed and q^ / k^ are re-formed where needed --------------------------
    const u32x4 qraw = *reinterpret_cast<const u32x4*>(p.q + (tokc * H + h) * DK + c0);
    const u32x4 kraw = *reinterpret_cast<const u32x4*>(p.k + (tokc * H + h) * DK + c0);
    HvRaw hraw;
    HdhOps ops;
    load_ops(h * rep, ops);
    load_hv(h * rep, hraw);
    float rq = 1.f, rk = 1.f;
    if (p.use_l2norm) {
        float qv[8], kv[8];
        unpack8(qraw, qv);
        unpack8(kraw, kv);
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
    // q^ and k^ as the forward rounds them (bf16 after the l2norm)
    // (zero in rows past the last token)
    auto qk_hat = [&](float (&qn)[8], float (&kn)[8]) {
        unpack8(qraw, qn);
        unpack8(kraw, kn);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (p.use_l2norm) {
                qn[j] = round_bf(qn[j] * rq);
                kn[j] = round_bf(kn[j] * rk);
            }
            qn[j] = valid ? qn[j] : 0.f;
            kn[j] = valid ? kn[j] : 0.f;
        }
    };
    float dQN[8], dKN[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) dQN[j] = dKN[j] = 0.f;

    const int nrep = GROUP ? rep : 1;
    for (int gi = 0; gi < nrep; ++gi) {
        const int hv = h * rep + gi;
        if (gi > 0) {
            load_ops(hv, ops);
            load_hv(hv, hraw);
        }
        HvRow hr;
        decode_hv(hraw, hr);
        const SeqSpan sp = seq_span(p, seq * HV + hv);
        const int64_t rec = sp.rec0 + c;
        const int64_t vrow = (tok * HV + hv) * DK;  // v/g/dO element offset of row i

        // ---- phase 1: gates, cumsum, recentred operands; the matrix-op
        // operands of phase 2 are loaded meanwhile ---------------------------
        float beta = hr.beta;
        if (p.use_beta_sigmoid) beta = valid ? fast_sigmoid(hr.beta) : 0.f;
        const float ea = p.use_gate ? expf(hr.alog) : 0.f;
        {
            float gv[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float gg = p.use_gate ? p.lower_bound * fast_sigmoid(ea * hr.g[j]) : hr.g[j];
                gv[j] = valid ? gg : 0.f;
            }
            lds_put8(&sm.dqg[i][c0], gv);  // the gate, then its cumsum G
            lds_put8(&sm.dvn[i][c0], hr.dvn);
        }
        __syncthreads();
        if ((p.use_gate || p.g_log) && t < DK) {
            // all 16 rows of column t read first, so their reads overlap
            float col[BT];
#pragma unroll
            for (int r = 0; r < BT; ++r) col[r] = sm.dqg[r][t];
            float run = 0.f;
#pragma unroll
            for (int r = 0; r < BT; ++r) {
                run += col[r];
                sm.dqg[r][t] = run * RCP_LN2;
            }
        }
        __syncthreads();
        if (t < DK) {
            sm.el[t] = fast_exp2(sm.dqg[last][t]);
            sm.gm[t] = sm.dqg[mid][t];
            sm.gl[t] = sm.dqg[last][t];
        }
        // E = 2^G, the recentred 2^(G - G_mid), 2^(G_mid - G), and
        // 2^(G_last - G), from this row's G and the rows mid and last
        float G[8];
        lds_get8(&sm.dqg[i][c0], G);
        auto gates = [&](float (&E)[8], float (&eq)[8], float (&ek)[8], float (&kgl)[8]) {
            float Gm[8], Gl[8];
            lds_get8(&sm.gm[c0], Gm);
            lds_get8(&sm.gl[c0], Gl);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                E[j] = valid ? fast_exp2(G[j]) : 0.f;
                eq[j] = valid ? fast_exp2(G[j] - Gm[j]) : 0.f;
                ek[j] = valid ? fast_exp2(Gm[j] - G[j]) : 0.f;
                kgl[j] = valid ? fast_exp2(Gl[j] - G[j]) : 0.f;
            }
        };
        __syncthreads();  // gm, gl
        {
            float E[8], eq[8], ek[8], kgl[8], qn[8], kn[8], o1[8], o2[8], o3[8], o4[8], o5[8];
            gates(E, eq, ek, kgl);
            qk_hat(qn, kn);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                o1[j] = qn[j] * eq[j];
                o2[j] = kn[j] * eq[j];
                o3[j] = kn[j] * ek[j];
                o4[j] = round_bf(round_bf(kn[j] * beta) * E[j]);
                o5[j] = round_bf(hr.v[j] * beta);
            }
            lds_put8(&sm.qp[i][c0], o1);
            lds_put8(&sm.kp[i][c0], o2);
            lds_put8(&sm.km[i][c0], o3);
            lds_put8_bf(&sm.kb[i][c0], o4);
            lds_put8_bf(&sm.vb[i][c0], o5);
        }
        __syncthreads();  // G is read; phase 2 overwrites dqg

        // ---- phase 2: products over V on the matrix cores ----------------
        mask_ops(ops);
        // Wave w owns k-tiles 2w, 2w+1.  Lane (x, q4) feeds row x of dO /
        // dv_new / v_new and row 16*kt + x of h / dh', v columns
        // 32*jv + 8*q4 .. +7, as 16x16x32 operands.
        {
            f32x4 aq[2], aw[2], ak[2], adq = {0.f, 0.f, 0.f, 0.f};
            float pel[2] = {0.f, 0.f};
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) aq[tt] = aw[tt] = ak[tt] = adq;
#pragma unroll
            for (int jv = 0; jv < 4; ++jv) {
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
                    const u32x4 bh = ops.bh[jv][tt], bd = ops.bd[jv][tt];
                    aq[tt] = mfma_bf16_16x16x32(as_bf16x8(ops.a_do[jv]), as_bf16x8(bh), aq[tt]);
                    aw[tt] = mfma_bf16_16x16x32(as_bf16x8(ops.a_dv[jv]), as_bf16x8(bh), aw[tt]);
                    ak[tt] = mfma_bf16_16x16x32(as_bf16x8(ops.a_vn[jv]), as_bf16x8(bd), ak[tt]);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        pel[tt] = fmaf(__builtin_bit_cast(float, bh[e] << 16),
                                       __builtin_bit_cast(float, bd[e] << 16), pel[tt]);
                        pel[tt] = fmaf(__builtin_bit_cast(float, bh[e] & 0xffff0000u),
                                       __builtin_bit_cast(float, bd[e] & 0xffff0000u), pel[tt]);
                    }
                }
                if (w == 0)
                    adq = mfma_bf16_16x16x32(as_bf16x8(ops.a_do[jv]), as_bf16x8(ops.a_vn[jv]), adq);
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
                float s2 = pel[tt];
                s2 += xor16(s2);
                s2 += __shfl_xor(s2, 32);
                if (q4 == 0) sm.del[16 * kt + x] = s2;
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

        // ---- phase 3: dA = dw kb^T + du vb^T, four partial sums in the
        // 16x16 scratch (wave w: dw (w < 2) or du, columns 64 (w & 1) ..
        // +63).  The gram Lraw = kp km^T and A_inv = (I + L)^-1
        // (kernels.py:157-167) come from stage 1's record, as the forward
        // formed them, instead of a second gram and solve here ------------
        {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            const int c64 = 64 * (w & 1);
            if (w < 2) {
#pragma unroll
                for (int sl = 0; sl < 16; ++sl) {
                    const int col = c64 + 4 * sl + q4;
                    acc = mfma_f32_16x16x4(sm.dw[x][col], bf2f(sm.kb[x][col]), acc);
                }
            } else {
#pragma unroll
                for (int sl = 0; sl < 16; ++sl) {
                    const int col = c64 + 4 * sl + q4;
                    acc = mfma_f32_16x16x4(sm.dvn[x][col], bf2f(sm.vb[x][col]), acc);
                }
            }
            float (*part)[BT + 1] = w == 0 ? sm.m1 : w == 1 ? sm.dlr : w == 2 ? sm.da : sm.lraw;
#pragma unroll
            for (int e = 0; e < 4; ++e) part[4 * q4 + e][x] = acc[e];
        }
        __syncthreads();
        {
            const float da = (sm.m1[i][cb] + sm.dlr[i][cb]) + (sm.da[i][cb] + sm.lraw[i][cb]);
            sm.da[i][cb] = da;
            sm.lraw[i][cb] = hraw.lraw;
            sm.ainv[i][cb] = hraw.ainv;
        }
        __syncthreads();

        // ---- phase 4: dkb = A^T dw, dvb = A^T du (A = bf16(A_inv), the
        // operand of w and u, kernels.py:170), dA A^T ------------------------
        f32x4 dkbt[2], dvbt[2];
        {
            float s2 = 0.f;
#pragma unroll
            for (int m = 0; m < BT; ++m) s2 = fmaf(sm.da[i][m], sm.ainv[cb][m], s2);
            sm.m1[i][cb] = s2;  // (dA A^T)[i][cb]; m1 is free after the partial sums
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                const int col = 16 * (2 * w + tt) + x;
                dkbt[tt] = dvbt[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int sl = 0; sl < 4; ++sl) {
                    const int r = 4 * sl + q4;
                    const float a = round_bf(sm.ainv[r][x]);
                    dkbt[tt] = mfma_f32_16x16x4(a, sm.dw[r][col], dkbt[tt]);
                    dvbt[tt] = mfma_f32_16x16x4(a, sm.dvn[r][col], dvbt[tt]);
                }
            }
        }
        __syncthreads();

        // ---- phase 5: dL = -A^T dA A^T (strictly lower), dLr = beta dL; the
        // dkb / dvb tiles replace dw / du (read for the last time above) ----
        float dbl;
        {
            float s2 = 0.f;
#pragma unroll
            for (int m = 0; m < BT; ++m) s2 = fmaf(sm.ainv[m][i], sm.m1[m][cb], s2);
            const float dl = (i > cb) ? -s2 : 0.f;
            sm.dlr[i][cb] = beta * dl;
            dbl = row_sum16(dl * sm.lraw[i][cb]);
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                const int col = 16 * (2 * w + tt) + x;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    sm.dw[4 * q4 + e][col] = dkbt[tt][e];
                    sm.dvn[4 * q4 + e][col] = dvbt[tt][e];
                }
            }
        }
        __syncthreads();

        // ---- phase 6: dkp = dLr km, dqp = dAqm km, dkm = dLr^T kp + dAqm^T qp
        // on the matrix cores, each wave its two column tiles, written in
        // place of kp / qp / km (only this wave reads those columns) --------
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int col = 16 * (2 * w + tt) + x;
            f32x4 dkp = {0.f, 0.f, 0.f, 0.f}, dqp = dkp, dkm = dkp;
#pragma unroll
            for (int sl = 0; sl < 4; ++sl) {
                const int r = 4 * sl + q4;
                const float kmv = sm.km[r][col];
                dkp = mfma_f32_16x16x4(sm.dlr[x][r], kmv, dkp);
                dqp = mfma_f32_16x16x4(sm.daqm[x][r], kmv, dqp);
                dkm = mfma_f32_16x16x4(sm.dlr[r][x], sm.kp[r][col], dkm);
                dkm = mfma_f32_16x16x4(sm.daqm[r][x], sm.qp[r][col], dkm);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                sm.kp[4 * q4 + e][col] = dkp[e];
                sm.qp[4 * q4 + e][col] = dqp[e];
                sm.km[4 * q4 + e][col] = dkm[e];
            }
        }
        __syncthreads();

        // ---- phase 7: the row-wise gradients ------------------------------
        float dG[8];
        {
            float dkp[8], dqp[8], dkm[8], dkb[8], dvb[8], dqg[8], dkg[8], dv[8];
            float E[8], eq[8], ek[8], kgl[8], qn[8], kn[8];
            gates(E, eq, ek, kgl);
            qk_hat(qn, kn);
            lds_get8(&sm.kp[i][c0], dkp);
            lds_get8(&sm.qp[i][c0], dqp);
            lds_get8(&sm.km[i][c0], dkm);
            lds_get8(&sm.dw[i][c0], dkb);
            lds_get8(&sm.dvn[i][c0], dvb);
            lds_get8(&sm.dqg[i][c0], dqg);
            lds_get8(&sm.dkg[i][c0], dkg);
            float dbeta = 0.f, kgkg[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float qp = qn[j] * eq[j], kp = kn[j] * eq[j], km = kn[j] * ek[j];
                const float qg = qn[j] * E[j], kg = kn[j] * kgl[j];
                const float kb = round_bf(round_bf(kn[j] * beta) * E[j]);
                dQN[j] += dqg[j] * E[j] + dqp[j] * eq[j];
                dKN[j] += dkb[j] * beta * E[j] + dkg[j] * kgl[j] + dkp[j] * eq[j] + dkm[j] * ek[j];
                dbeta = fmaf(dkb[j], kn[j] * E[j], dbeta);
                dbeta = fmaf(dvb[j], hr.v[j], dbeta);
                dv[j] = dvb[j] * beta;
                const float d = LN2 * (dkb[j] * kb + dqg[j] * qg - dkg[j] * kg + dqp[j] * qp +
                                       dkp[j] * kp - dkm[j] * km);
                dG[j] = valid ? d : 0.f;
                kgkg[j] = valid ? dkg[j] * kg : 0.f;
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
            // kp and km (dkp, dkm) are read only by their owning thread here
            lds_put8(&sm.kp[i][c0], dG);
            lds_put8(&sm.km[i][c0], kgkg);
        }
        __syncthreads();

        // ---- phase 8: the last row's dG (through kg and the state decay),
        // then per row the reverse cumsum of dG into dgate and the gate
        // (kernels.py:115-124) -------------------------------------------
        // One pass per column: the last row's terms, then the suffix sums
        // over the valid rows into the dead dw tile (all 16 rows of the
        // column read first, so their reads overlap).
        if (t < DK) {
            float s2 = 0.f, col[BT];
#pragma unroll
            for (int r = 0; r < BT; ++r) {
                s2 += sm.km[r][t];
                col[r] = sm.kp[r][t];
            }
            const float lastterm = LN2 * (s2 + sm.el[t] * sm.del[t]);
            float run = 0.f;
#pragma unroll
            for (int r = BT - 1; r >= 0; --r) {
                if (r == last) col[r] += lastterm;
                if (r < nvalid) run += col[r];
                sm.dw[r][t] = r < nvalid ? run : 0.f;
                if (r == last) sm.kp[r][t] = col[r];
            }
        }
        __syncthreads();
        {
            float dg[8], suf[8], own[8];
            lds_get8(&sm.kp[i][c0], own);  // dG with the last row's terms
            lds_get8(&sm.dw[i][c0], suf);  // its suffix sum over rows >= i
            float pdt[8], pal[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float d;
                if (p.use_gate) {
                    const float sarg = hr.g[j];
                    const float sg = fast_sigmoid(ea * sarg);
                    d = RCP_LN2 * suf[j] * p.lower_bound * sg * (1.f - sg) * ea;
                    pdt[j] = valid ? d : 0.f;
                    pal[j] = valid ? d * sarg : 0.f;
                } else if (p.g_log) {
                    d = RCP_LN2 * suf[j];
                } else {
                    d = own[j];
                }
                dg[j] = d;
            }
            if (valid) {
                if (p.g_bf16) {
                    store8(static_cast<uint16_t*>(p.dg) + vrow + c0, dg);
                } else {
                    float* dst = static_cast<float*>(p.dg) + vrow + c0;
                    *reinterpret_cast<f32x4*>(dst) = f32x4{dg[0], dg[1], dg[2], dg[3]};
                    *reinterpret_cast<f32x4*>(dst + 4) = f32x4{dg[4], dg[5], dg[6], dg[7]};
                }
            }
            if (gate_grads) {
                // column sums for ddt_bias, dA_log's terms, through the dead
                // qp / dqg tiles
                lds_put8(&sm.qp[i][c0], pdt);
                lds_put8(&sm.dqg[i][c0], pal);
            }
        }
        if (gate_grads) {
            __syncthreads();
            if (t < DK) {
                float sdt = 0.f, sal = 0.f;
#pragma unroll
                for (int r = 0; r < BT; ++r) {
                    sdt += sm.qp[r][t];
                    sal += sm.dqg[r][t];
                }
                p.tr_part[rec * PART_STRIDE + t] = sdt;
                sal = row_sum16(sal);
                sal += xor16(sal);
                sal += __shfl_xor(sal, 32);
                if (lane == 0) sm.red[w] = sal;
            }
            __syncthreads();
            if (t == 0) p.tr_part[rec * PART_STRIDE + DK] = sm.red[0] + sm.red[1];
        }
        __syncthreads();
    }

    // ---- l2norm backward, dq / dk summed over the group -------------------
    if (p.use_l2norm) {
        float qv[8], kv[8];
        unpack8(qraw, qv);
        unpack8(kraw, kv);
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
// head hv (PART_STRIDE floats per record: DK bias sums, then the A_log
// sum), in a fixed order, in two launches:
//   1. the head's records (its batch rows' runs, or its varlen slots, in
//      order) fall into segments of GR_SEG consecutive records, one
//      work-group each: thread group j (of RG) sums records j, j + RG, ...
//      of the segment, then the groups' sums are added in group order, and
//      the segment's sum replaces its first record's partials (read by then);
//   2. one work-group per head adds its segments' sums in segment order.
// The order depends on the geometry only, so the sums are bit for bit
// repeatable.
constexpr int RG = 8;
constexpr int GR_SEG = 32;

// Records of value head hv: nb runs of nr, run b starting at first(b).
struct GateRuns {
    int nb, nr;
    __device__ __forceinline__ GateRuns(const Params& p)
        : nb(p.cu_seqlens ? 1 : p.B), nr(p.cu_seqlens ? p.NS : p.NT) {}
    __device__ __forceinline__ float* rec(const Params& p, int hv, int i) const {
        const int b = i / nr, x = i - b * nr;
        const int64_t first = p.cu_seqlens ? (int64_t)hv * p.NS : (int64_t)(b * p.HV + hv) * p.NT;
        return p.tr_part + (first + x) * PART_STRIDE;
    }
};

__global__ __launch_bounds__(RG * DK) void gate_segment_kernel(Params p) {
    __shared__ float s_acc[RG][DK + 1];
    const GateRuns runs(p);
    const int nrec = runs.nb * runs.nr;
    const int nseg = (nrec + GR_SEG - 1) / GR_SEG;
    const int hv = blockIdx.x / nseg, seg = blockIdx.x - hv * nseg;
    const int t = threadIdx.x & (DK - 1), grp = threadIdx.x / DK;
    const int i0 = seg * GR_SEG, i1 = min(i0 + GR_SEG, nrec);
    float acc = 0.f, accA = 0.f;
    // the segment's loads in flight before the adds, which keep their order
#pragma unroll 4
    for (int i = i0 + grp; i < i1; i += RG) {
        const float* r = runs.rec(p, hv, i);
        acc += r[t];
        if (t == 0) accA += r[DK];
    }
    s_acc[grp][t] = acc;
    if (t == 0) s_acc[grp][DK] = accA;
    __syncthreads();  // every read of the segment's records is done
    if (grp == 0) {
        float a = 0.f;
#pragma unroll
        for (int j = 0; j < RG; ++j) a += s_acc[j][t];
        float* out = runs.rec(p, hv, i0);
        out[t] = a;
        if (t == 0) {
            float aa = 0.f;
#pragma unroll
            for (int j = 0; j < RG; ++j) aa += s_acc[j][DK];
            out[DK] = aa;
        }
    }
}

__global__ __launch_bounds__(DK) void gate_reduce_kernel(Params p) {
    const GateRuns runs(p);
    const int nrec = runs.nb * runs.nr;
    const int hv = blockIdx.x, t = threadIdx.x;
    float a = 0.f, aa = 0.f;
    // sixteen segments' loads in flight before their adds (in order)
#pragma unroll 16
    for (int i0 = 0; i0 < nrec; i0 += GR_SEG) {
        const float* r = runs.rec(p, hv, i0);
        a += r[t];
        if (t == 0) aa += r[DK];
    }
    if (p.ddt_bias) p.ddt_bias[hv * DK + t] = a;
    if (t == 0 && p.dA_log) p.dA_log[hv] = aa;
}

}  // namespace

hipError_t launch_bwd_chunk(const Params& p, hipStream_t stream) {
    const int64_t grid = p.cu_seqlens ? (int64_t)p.H * p.NS : (int64_t)p.B * p.H * p.NT;
    const bool full = !p.cu_seqlens && p.T % BT == 0;
    auto kern = p.HV > p.H ? (full ? bwd_chunk_kernel<true, true> : bwd_chunk_kernel<true, false>)
                           : (full ? bwd_chunk_kernel<false, true> : bwd_chunk_kernel<false, false>);
    hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(CT), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_bwd_gate_reduce(const Params& p, hipStream_t stream) {
    const int64_t nrec = p.cu_seqlens ? (int64_t)p.NS : (int64_t)p.B * p.NT;
    const int64_t nseg = (nrec + GR_SEG - 1) / GR_SEG;
    if (nseg > 0) {
        hipLaunchKernelGGL(gate_segment_kernel, dim3((unsigned)(p.HV * nseg)), dim3(RG * DK), 0, stream, p);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(gate_reduce_kernel, dim3((unsigned)p.HV), dim3(DK), 0, stream, p);
    return hipGetLastError();
}

}  // namespace kda
