// Stage 2 of the KDA BT=16 forward: the serial delta-rule recurrence.
//
// Follows kda_bt16_kernel_k2 (/root/reference/src/kda_bt16/kernels.py:187-302):
// per chunk,
//   hc    = bf16(S)
//   v_new = bf16(u - w @ hc^T)
//   o     = bf16(scale * (qg @ hc^T) + Aqk @ v_new)
//   S     = S * 2^G_last[None, :] + (kg^T @ v_new)^T
// with S the [V, K] fp32 state.  One 64-lane wave owns 16 value columns of
// one (batch, head) and keeps its slice of S transposed, S^T[k][v], as eight
// 16x16 fp32 accumulator tiles.  The 16x16 accumulator layout (lane
// v + 16*(k/4), item k%4) is exactly the B-operand layout of the 16x16x16
// bf16 matrix op, so bf16(S) feeds the next chunk's products straight from
// registers: the serial chain itself never goes through LDS.  Pairs of
// k-tiles form the 8-deep operands of the 16x16x32 op for w @ hc^T and
// qg @ hc^T; stage 1 stored w and qg in the matching k order.
#include "kda_common.h"

namespace kda {

namespace {

// Records stream through an LDS ring of RING slots with the gfx950 direct
// global->LDS loads (buffer_load_dwordx4 ... lds: 16 B per lane, 1 KiB per
// wave instruction), issued RING-1 chunks ahead of use.  A wave copies the
// 13 KiB every value tile needs plus the 1 KiB pair of u slices that holds
// its own 512-byte slice: 14 loads per chunk.  The loads complete in issue
// order, so before reading a slot the wave waits until at most
// 14 * (chunks issued after it) loads are outstanding; stores counted in the
// same counter only lengthen that wait.  A wave may have at most 63 vector
// memory operations in flight (the vmcnt field is 6 bits) before issue
// stalls: (RING - 1) * 14 loads plus the step's single store stay below.
constexpr int RING = 5;
constexpr int SHARED_LOADS = REC_SHARED / 1024;
constexpr int LOADS_PER_CHUNK = SHARED_LOADS + 1;
constexpr int SLOT = REC_SHARED + 1024;
static_assert(SHARED_LOADS * 1024 == REC_SHARED, "shared part must be whole KiB");
static_assert((RING - 1) * LOADS_PER_CHUNK + 1 <= 63, "vmcnt is a 6-bit count");

typedef __attribute__((address_space(3))) uint8_t lds_u8;

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Wait until the chunk followed by `n_after` issued chunks has landed.
__device__ __forceinline__ void wait_chunk(int n_after) {
    static_assert(RING == 5, "ladder below covers 0..4 later chunks");
    if (n_after >= 4) {
        wait_vmcnt<4 * LOADS_PER_CHUNK>();
    } else if (n_after == 3) {
        wait_vmcnt<3 * LOADS_PER_CHUNK>();
    } else if (n_after == 2) {
        wait_vmcnt<2 * LOADS_PER_CHUNK>();
    } else if (n_after == 1) {
        wait_vmcnt<LOADS_PER_CHUNK>();
    } else {
        wait_vmcnt<0>();
    }
}

// Buffer descriptor word 3 for raw byte-addressed buffers on gfx9-family
// parts (gfx950 included).
constexpr int BUF_DWORD3 = 0x00020000;

// Loads [I0, I1) of one chunk's copy; index SHARED_LOADS is the 1 KiB pair
// of u slices (value tiles 2*(vt/2) and 2*(vt/2)+1), always inside the
// record.  Buffer loads with the chunk offset in an SGPR and a fixed
// per-lane VGPR offset: no per-step address arithmetic on the vector ALU.
template <int I0, int I1>
__device__ __forceinline__ void issue_part(__amdgpu_buffer_rsrc_t rs, uint32_t chunk_off,
                                           lds_u8* slot, int vt, uint32_t voff16) {
#pragma unroll
    for (int i = I0; i < I1; ++i) {
        const uint32_t src = i < SHARED_LOADS ? chunk_off + i * 1024
                                              : chunk_off + REC_U + (uint32_t)(vt >> 1) * 1024;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_u8*)(slot + i * 1024), 16, voff16, src,
                                                 0, 0);
    }
}

__device__ __forceinline__ void issue_chunk(__amdgpu_buffer_rsrc_t rs, uint32_t chunk_off,
                                            lds_u8* slot, int vt, uint32_t voff16) {
    issue_part<0, LOADS_PER_CHUNK>(rs, chunk_off, slot, vt, voff16);
}

// One chunk's operands in registers, read from the ring one step ahead.
// Every ring read sits right after the explicit wait for its chunk: the
// compiler cannot tell ring slots apart, and a ring read that follows a
// direct-to-LDS load issue without such a wait gets a conservative
// vmcnt(0) from it, which would stall every step on the newest load.
struct Ops {
    u32x4 w[4];
    u32x4 qg[4];
    u32x4 kg[4];
    f32x4 dc[8];
    u32x2 aqk;
    u32x2 u;
};

__device__ __forceinline__ void read_ops(const uint8_t* slot, int lane, int q4, int vt, Ops& op) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
        op.w[j] = *reinterpret_cast<const u32x4*>(slot + REC_W + j * 1024 + lane * 16);
    op.u = *reinterpret_cast<const u32x2*>(slot + REC_SHARED + (vt & 1) * 512 + lane * 8);
    op.aqk = *reinterpret_cast<const u32x2*>(slot + REC_AQK + lane * 8);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        op.qg[j] = *reinterpret_cast<const u32x4*>(slot + REC_QG + j * 1024 + lane * 16);
        op.kg[j] = *reinterpret_cast<const u32x4*>(slot + REC_KG + j * 1024 + lane * 16);
    }
#pragma unroll
    for (int kt = 0; kt < 8; ++kt)
        op.dc[kt] = *reinterpret_cast<const f32x4*>(slot + REC_DECAY + kt * 64 + q4 * 16);
}

// The record ring (one per work-group).  Referenced by name everywhere, so
// every ring address is a known LDS offset; the direct loads take it as an
// LDS-space pointer, cast before any offset is applied.
__shared__ __attribute__((aligned(1024))) uint8_t ring[RING * SLOT];

__device__ __forceinline__ lds_u8* ring_lds() { return (lds_u8*)ring; }

// 4x4 transpose of 16-bit values across the 4 lanes of a quad.  Lane j
// enters with p0 = (M[0][j], M[1][j]) and p1 = (M[2][j], M[3][j]) and leaves
// with (M[j][0], M[j][1]) and (M[j][2], M[j][3]).  Two DPP exchanges:
// lanes j and j^2 swap the 2x2 blocks off the diagonal, then lanes j and
// j^1 swap 16-bit halves.
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

// Per-wave constants of the chunk loop.
struct Ctx {
    __amdgpu_buffer_rsrc_t rs;  // this head's records, NT * REC_BYTES bytes
    uint32_t voff16;            // lane * 16
    uint16_t* obase;     // o[b, 0, h, 16*vt + 4*((lane%16)/4)]
    int64_t orow_stride; // elements between consecutive tokens of o
    float scale;
    int NT, T, lane, q4, x, vt;
};

// One chunk of the recurrence.  S (the ring slot of chunk c) is a template
// argument so that every ring offset is a compile-time constant: alias
// analysis then sees that the slot being refilled, the slot being read and
// the slot being prefetched are disjoint, and no conservative wait on the
// newest direct-to-LDS load is inserted.
template <int S>
__device__ __forceinline__ void chunk_step(const Ctx& cx, int c, f32x4 (&St)[8], Ops& cur) {
    // The copy of chunk c + RING - 1 goes out in three groups spread over
    // the step, so the address unit drains them while the matrix ops run
    // instead of stalling the wave on back-to-back issue.
    const int cn = c + RING - 1;
    const bool refill = cn < cx.NT;
    const uint32_t src = (uint32_t)cn * REC_BYTES;
    lds_u8* dst = ring_lds() + ((S + RING - 1) % RING) * SLOT;
    if (refill) issue_part<0, 5>(cx.rs, src, dst, cx.vt, cx.voff16);

    // hc = bf16(S), as 16x16x32 B operands (k-tiles 2j and 2j+1).
    bf16x8 hc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const u32x4 pk = {pack2(St[2 * j][0], St[2 * j][1]), pack2(St[2 * j][2], St[2 * j][3]),
                          pack2(St[2 * j + 1][0], St[2 * j + 1][1]),
                          pack2(St[2 * j + 1][2], St[2 * j + 1][3])};
        hc[j] = as_bf16x8(pk);
    }
    // v_new = u - w @ hc^T, two independent accumulation chains
    // (kernels.py:261-266), rounded to bf16.
    const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
    f32x4 va = mfma_bf16_16x16x32(as_bf16x8(cur.w[0]), hc[0], zero);
    f32x4 vb = mfma_bf16_16x16x32(as_bf16x8(cur.w[2]), hc[2], zero);
    va = mfma_bf16_16x16x32(as_bf16x8(cur.w[1]), hc[1], va);
    vb = mfma_bf16_16x16x32(as_bf16x8(cur.w[3]), hc[3], vb);
    f32x4 oacc = mfma_bf16_16x16x32(as_bf16x8(cur.qg[0]), hc[0], zero);
#pragma unroll
    for (int j = 1; j < 4; ++j) oacc = mfma_bf16_16x16x32(as_bf16x8(cur.qg[j]), hc[j], oacc);
    if (refill) issue_part<5, 10>(cx.rs, src, dst, cx.vt, cx.voff16);
    const f32x4 vacc = va + vb;
    const float u0 = __builtin_bit_cast(float, cur.u.x << 16);
    const float u1 = __builtin_bit_cast(float, cur.u.x & 0xffff0000u);
    const float u2 = __builtin_bit_cast(float, cur.u.y << 16);
    const float u3 = __builtin_bit_cast(float, cur.u.y & 0xffff0000u);
    const u32x2 vnb = {pack2(u0 - vacc[0], u1 - vacc[1]), pack2(u2 - vacc[2], u3 - vacc[3])};
    const i16x4 vn = as_i16x4(vnb);

    // S = S * 2^G_last + (kg^T @ v_new)^T (kernels.py:281-294).
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const u32x2 k0 = {cur.kg[j].x, cur.kg[j].y};
        const u32x2 k1 = {cur.kg[j].z, cur.kg[j].w};
        St[2 * j] = mfma_bf16_16x16x16(as_i16x4(k0), vn, St[2 * j] * cur.dc[2 * j]);
        St[2 * j + 1] = mfma_bf16_16x16x16(as_i16x4(k1), vn, St[2 * j + 1] * cur.dc[2 * j + 1]);
    }

    // o = scale * qg @ hc^T + Aqk @ v_new (kernels.py:268-279).
    oacc = oacc * cx.scale;
    oacc = mfma_bf16_16x16x16(as_i16x4(cur.aqk), vn, oacc);
    if (refill) issue_part<10, LOADS_PER_CHUNK>(cx.rs, src, dst, cx.vt, cx.voff16);

    // Operands of the next chunk: wait for its copy, read them while the
    // matrix ops above drain.
    if (c + 1 < cx.NT) {
        wait_chunk(min(RING - 2, cx.NT - 2 - c));
        read_ops(ring + ((S + 1) % RING) * SLOT, cx.lane, cx.q4, cx.vt, cur);
    }

    // o: lane (x = 4a + b, q4) holds o[4*q4 + i][16*vt + x], i = 0..3.  A
    // 4x4 transpose of 16-bit values inside each quad of lanes leaves lane b
    // with row 4*q4 + b, columns 4a..4a+3: one 8-byte store per lane.
    const u32x2 ot = quad_transpose(pack2(oacc[0], oacc[1]), pack2(oacc[2], oacc[3]), cx.lane & 3);
    const int t = c * BT + 4 * cx.q4 + (cx.lane & 3);
    if (t < cx.T) *reinterpret_cast<u32x2*>(cx.obase + (int64_t)t * cx.orow_stride) = ot;
}

__global__ __launch_bounds__(64) void k2_kernel(Params p) {

    const int lane = threadIdx.x;
    const int x = lane & 15;  // value column inside the tile
    const int q4 = lane >> 4;
    const int H = p.H, T = p.T, NT = p.NT;
    const int nbh = p.B * H;

    // Work-group -> (head, value tile), XCD aware: consecutive work-group ids
    // go to different XCDs round-robin, so the 8 tiles of one head get ids
    // of one residue class mod 8 and share that XCD's L2 for the records.
    const int wg = blockIdx.x;
    const int lin = (wg & 7) * nbh + (wg >> 3);
    const int bh = lin >> 3;
    const int vt = lin & 7;
    const int b = bh / H, h = bh - (bh / H) * H;
    const int v = 16 * vt + x;

    // S^T tiles: St[kt][i] = S[v][16*kt + 4*q4 + i].
    f32x4 St[8];
    const int64_t sbase = (int64_t)bh * DK * DK;
#pragma unroll
    for (int kt = 0; kt < 8; ++kt) {
        St[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (p.h0) {
            const int k0 = 16 * kt + 4 * q4;
            if (p.h0_v_first) {
                St[kt] = *reinterpret_cast<const f32x4*>(p.h0 + sbase + (int64_t)v * DK + k0);
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) St[kt][i] = p.h0[sbase + (int64_t)(k0 + i) * DK + v];
            }
        }
    }

    Ctx cx;
    cx.rs = __builtin_amdgcn_make_buffer_rsrc(p.ws + (int64_t)bh * NT * REC_BYTES, (short)0,
                                              NT * REC_BYTES, BUF_DWORD3);
    cx.voff16 = lane * 16;
    cx.obase = p.o + ((int64_t)b * T * H + h) * DK + 16 * vt + 4 * (x >> 2);
    cx.orow_stride = (int64_t)H * DK;
    cx.scale = p.scale;
    cx.NT = NT;
    cx.T = T;
    cx.lane = lane;
    cx.q4 = q4;
    cx.x = x;
    cx.vt = vt;

#pragma unroll
    for (int d = 0; d < RING - 1; ++d)
        if (d < NT)
            issue_chunk(cx.rs, (uint32_t)d * REC_BYTES, ring_lds() + d * SLOT, vt, cx.voff16);
    wait_chunk(min(RING - 2, NT - 1));
    Ops cur;
    read_ops(ring, lane, q4, vt, cur);

    static_assert(RING == 5, "the unrolled loop below names every slot");
    for (int c = 0; c < NT; c += RING) {
        chunk_step<0>(cx, c, St, cur);
        if (c + 1 < NT) chunk_step<1>(cx, c + 1, St, cur);
        if (c + 2 < NT) chunk_step<2>(cx, c + 2, St, cur);
        if (c + 3 < NT) chunk_step<3>(cx, c + 3, St, cur);
        if (c + 4 < NT) chunk_step<4>(cx, c + 4, St, cur);
    }

    if (p.ht) {
#pragma unroll
        for (int kt = 0; kt < 8; ++kt) {
            const int k0 = 16 * kt + 4 * q4;
            if (p.ht_v_first) {
                *reinterpret_cast<f32x4*>(p.ht + sbase + (int64_t)v * DK + k0) = St[kt];
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) p.ht[sbase + (int64_t)(k0 + i) * DK + v] = St[kt][i];
            }
        }
    }
}

}  // namespace

hipError_t launch_k2(const Params& p, hipStream_t stream) {
    const int64_t grid = (int64_t)p.B * p.H * 8;
    hipLaunchKernelGGL(k2_kernel, dim3((unsigned)grid), dim3(64), 0, stream, p);
    return hipGetLastError();
}

}  // namespace kda
