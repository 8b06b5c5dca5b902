// C ABI of libkda_bt16_hip.so: argument checks, the two stage launches and
// the token recurrence.
// The checks here guard the kernels' indexing assumptions (shapes, pointer
// presence, workspace size, 32-bit grids); the user-facing validation with
// the reference's messages lives in the Python layer.
#include "../../include/kda_bt16_hip.h"
#include "kda_common.h"

#include <mutex>

namespace {

using kda::Params;

constexpr int64_t I32_MAX = 0x7fffffffLL;

bool misaligned(const void* p, uintptr_t align) {
    return (reinterpret_cast<uintptr_t>(p) & (align - 1)) != 0;
}

bool gate_dtype_ok(int32_t t) { return t == KDA_BT16_DTYPE_F32 || t == KDA_BT16_DTYPE_BF16; }

int64_t chunks_of(int64_t T) { return (T + kda::BT - 1) / kda::BT; }

// Sequences of the batch: B rows, or N packed sequences with cu_seqlens.
int64_t sequences(const KdaBt16Args* a) { return a->cu_seqlens ? a->N : a->B; }

// Record slots per value head with cu_seqlens: sequence n's chunks sit at
// floor(cu_seqlens[n] / 16) + n + c, all below floor(T / 16) + N.
int64_t varlen_slots(const KdaBt16Args* a) { return (int64_t)a->T / kda::BT + a->N; }

// Checks shared by every entry point and the common part of Params.
int check_common(const KdaBt16Args* a, Params& p) {
    if (a == nullptr) return KDA_BT16_EINVAL;
    if (a->abi_version != KDA_BT16_ABI_VERSION) return KDA_BT16_EABI;
    if (a->B <= 0 || a->T <= 0 || a->H <= 0 || a->HV <= 0 || a->K <= 0 || a->V <= 0)
        return KDA_BT16_EINVAL;
    if (a->K != kda::DK || a->V != kda::DK || a->HV % a->H != 0) return KDA_BT16_EUNSUPPORTED;
    if (!gate_dtype_ok(a->g_dtype) || !gate_dtype_ok(a->beta_dtype)) return KDA_BT16_EINVAL;
    if (a->cu_seqlens) {
        // Packed sequences: one batch row; 32- or 64-bit offsets.
        if (a->B != 1 || a->N <= 0) return KDA_BT16_EINVAL;
        if (a->cu_seqlens_dtype == KDA_BT16_DTYPE_I32) {
            if (misaligned(a->cu_seqlens, 4)) return KDA_BT16_EINVAL;
        } else if (a->cu_seqlens_dtype == KDA_BT16_DTYPE_I64) {
            if (misaligned(a->cu_seqlens, 8)) return KDA_BT16_EINVAL;
        } else {
            return KDA_BT16_EINVAL;
        }
    }
    const bool use_gate = (a->flags & KDA_BT16_USE_GATE) != 0;
    if (use_gate && !(a->lower_bound > -11.0f && a->lower_bound < 0.0f)) return KDA_BT16_ERANGE;

    p = Params{};
    p.q = static_cast<const uint16_t*>(a->q);
    p.k = static_cast<const uint16_t*>(a->k);
    p.v = static_cast<const uint16_t*>(a->v);
    p.g = a->g;
    p.beta = a->beta;
    p.A_log = a->A_log;
    p.dt_bias = a->dt_bias;
    p.h0 = a->h0;
    p.o = static_cast<uint16_t*>(a->o);
    p.ht = a->ht;
    p.B = a->B;
    p.T = a->T;
    p.tok_stride = a->T;
    p.H = a->H;
    p.HV = a->HV;
    p.NT = (int)chunks_of(a->T);
    p.scale = a->scale;
    p.lower_bound = a->lower_bound;
    p.g_bf16 = a->g_dtype == KDA_BT16_DTYPE_BF16;
    p.beta_bf16 = a->beta_dtype == KDA_BT16_DTYPE_BF16;
    p.use_gate = use_gate;
    p.use_l2norm = (a->flags & KDA_BT16_USE_QK_L2NORM) != 0;
    p.use_beta_sigmoid = (a->flags & KDA_BT16_USE_BETA_SIGMOID) != 0;
    p.g_log = (a->flags & KDA_BT16_G_LOG_DECAY) != 0;
    p.force_fused = (a->flags & KDA_BT16_FUSED_KERNEL) != 0;
    p.two_stage = (a->flags & KDA_BT16_TWO_STAGE) != 0;
    if (p.force_fused && p.two_stage) return KDA_BT16_EINVAL;
    if (a->k2_tiles != 0 && a->k2_tiles != 1 && a->k2_tiles != 2 && a->k2_tiles != 4 && a->k2_tiles != 8)
        return KDA_BT16_EINVAL;
    if (a->k2_wave_tiles < 0 || a->k2_wave_tiles > 2 || a->max_seqlen < 0) return KDA_BT16_EINVAL;
    p.k2_tiles = a->k2_tiles;
    p.k2_wave_tiles = a->k2_wave_tiles;
    p.max_seqlen = a->cu_seqlens ? a->max_seqlen : 0;
    p.h0_v_first = p.ht_v_first = (a->flags & KDA_BT16_STATE_V_FIRST) != 0;
    p.cu_seqlens = a->cu_seqlens;
    p.cu_i64 = a->cu_seqlens_dtype == KDA_BT16_DTYPE_I64;
    p.N = a->cu_seqlens ? a->N : 0;
    return KDA_BT16_OK;
}

// The chunked entries (stage 1, stage 2, both), all but the workspace.
int to_params_core(const KdaBt16Args* a, Params& p, bool need_inputs, bool need_outputs) {
    int rc = check_common(a, p);
    if (rc != KDA_BT16_OK) return rc;
    if (a->flags & KDA_BT16_O_FP32) return KDA_BT16_EUNSUPPORTED;
    // Grid sizes are 32-bit: stage 1 has one work-group per record slot,
    // stage 2 eight per (sequence, value head).  Stage 2 addresses one
    // sequence-head's records through a buffer descriptor with a 32-bit size
    // (at most ceil(T / 16) * REC_BYTES bytes).
    const int64_t slots = a->cu_seqlens ? varlen_slots(a) : (int64_t)a->B * chunks_of(a->T);
    if ((int64_t)a->HV * slots > I32_MAX || sequences(a) * a->HV * 8 > I32_MAX ||
        chunks_of(a->T) * kda::REC_BYTES > I32_MAX)
        return KDA_BT16_EUNSUPPORTED;
    p.NS = a->cu_seqlens ? (int)varlen_slots(a) : 0;
    if (need_inputs) {
        if (!a->q || !a->k || !a->v || !a->g || !a->beta) return KDA_BT16_EINVAL;
        if (p.use_gate && !a->A_log) return KDA_BT16_EINVAL;
        const bool any_dbg = a->dbg_Aqk || a->dbg_A_inv || a->dbg_w || a->dbg_u || a->dbg_g;
        const bool all_dbg = a->dbg_Aqk && a->dbg_A_inv && a->dbg_w && a->dbg_u && a->dbg_g;
        if (any_dbg && !all_dbg) return KDA_BT16_EINVAL;
    }
    if (need_outputs && !a->o) return KDA_BT16_EINVAL;
    // The kernels use 8- and 16-byte vector accesses.
    if (misaligned(a->q, 16) || misaligned(a->k, 16) || misaligned(a->v, 16) ||
        misaligned(a->g, 16) || misaligned(a->beta, a->beta_dtype == KDA_BT16_DTYPE_BF16 ? 2 : 4) ||
        misaligned(a->dt_bias, 16) ||
        misaligned(a->h0, 16) || misaligned(a->ht, 16) || misaligned(a->o, 16) ||
        misaligned(a->dbg_Aqk, 8) || misaligned(a->dbg_A_inv, 8) || misaligned(a->dbg_w, 16) ||
        misaligned(a->dbg_u, 16) || misaligned(a->dbg_g, 16))
        return KDA_BT16_EINVAL;
    p.dbg_Aqk = static_cast<uint16_t*>(a->dbg_Aqk);
    p.dbg_A_inv = static_cast<uint16_t*>(a->dbg_A_inv);
    p.dbg_w = static_cast<uint16_t*>(a->dbg_w);
    p.dbg_u = static_cast<uint16_t*>(a->dbg_u);
    p.dbg_g = a->dbg_g;
    return KDA_BT16_OK;
}

// The caller's workspace (for the records stage 1 hands to stage 2).
int take_workspace(const KdaBt16Args* a, Params& p) {
    const size_t need = kda_bt16_workspace_bytes_args(a);
    if (!a->workspace || a->workspace_bytes < need) return KDA_BT16_EWORKSPACE;
    if ((reinterpret_cast<uintptr_t>(a->workspace) & 255u) != 0) return KDA_BT16_EWORKSPACE;
    p.ws = static_cast<uint8_t*>(a->workspace);
    return KDA_BT16_OK;
}

// The chunked entries with the caller's workspace.
int to_params(const KdaBt16Args* a, Params& p, bool need_inputs, bool need_outputs) {
    int rc = to_params_core(a, p, need_inputs, need_outputs);
    if (rc != KDA_BT16_OK) return rc;
    return take_workspace(a, p);
}

// Scratch of kda_bt16_fwd_noalloc_hip: the records stage 1 hands to stage
// 2, in a file-scope device array instead of a caller's workspace.  In host
// code `scratch` names a host-side stand-in, never the device memory: the
// device address comes from hipGetSymbolAddress, once per device (each GPU
// holds its own copy of the array), and only that address is passed on.
__device__ __align__(256) static uint8_t scratch[KDA_BT16_NOALLOC_MAX_WORKSPACE];

constexpr int MAX_DEVICES = 64;
std::mutex scratch_mu;
uint8_t* scratch_dev[MAX_DEVICES] = {};

// The current device's address of `scratch` (looked up on the first call
// on that device, with that device current).
int scratch_ptr(uint8_t** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) return KDA_BT16_ELAUNCH;
    if (dev < 0 || dev >= MAX_DEVICES) return KDA_BT16_EUNSUPPORTED;
    std::lock_guard<std::mutex> lock(scratch_mu);
    if (scratch_dev[dev] == nullptr) {
        void* ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr)
            return KDA_BT16_ELAUNCH;
        if ((reinterpret_cast<uintptr_t>(ptr) & 255u) != 0) return KDA_BT16_ELAUNCH;
        scratch_dev[dev] = static_cast<uint8_t*>(ptr);
    }
    *out = scratch_dev[dev];
    return KDA_BT16_OK;
}

// The token recurrence: no workspace, no debug outputs, o in bf16 or fp32.
int to_params_recurrent(const KdaBt16Args* a, Params& p) {
    int rc = check_common(a, p);
    if (rc != KDA_BT16_OK) return rc;
    if (sequences(a) * a->HV > I32_MAX) return KDA_BT16_EUNSUPPORTED;
    if (!a->q || !a->k || !a->v || !a->g || !a->beta || !a->o) return KDA_BT16_EINVAL;
    if (p.use_gate && !a->A_log) return KDA_BT16_EINVAL;
    if (a->dbg_Aqk || a->dbg_A_inv || a->dbg_w || a->dbg_u || a->dbg_g) return KDA_BT16_EINVAL;
    // 16-byte state pieces; q, k, v and g rows read in 4-column pieces.
    if (misaligned(a->q, 16) || misaligned(a->k, 16) || misaligned(a->v, 16) ||
        misaligned(a->g, 16) ||
        misaligned(a->beta, a->beta_dtype == KDA_BT16_DTYPE_BF16 ? 2 : 4) ||
        misaligned(a->dt_bias, 4) || misaligned(a->h0, 16) || misaligned(a->ht, 16) ||
        misaligned(a->o, (a->flags & KDA_BT16_O_FP32) ? 4 : 2))
        return KDA_BT16_EINVAL;
    p.o_fp32 = (a->flags & KDA_BT16_O_FP32) != 0;
    return KDA_BT16_OK;
}

// Record slots of a geometry (every value head): B * HV * NT, or HV * NS.
int64_t record_slots(const KdaBt16Args* a) {
    return a->cu_seqlens ? (int64_t)a->HV * varlen_slots(a)
                         : (int64_t)a->B * a->HV * chunks_of(a->T);
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// Backward workspace regions, in order.
struct BwdLayout {
    size_t rec, brec, h, vn, dh, dvn, part, total;
};

BwdLayout bwd_layout(int64_t R) {
    BwdLayout L;
    size_t off = 0;
    L.rec = off;
    off = align256(off + (size_t)R * kda::REC_BYTES);
    L.brec = off;
    off = align256(off + (size_t)R * kda::REC_BYTES);
    L.h = off;
    off = align256(off + (size_t)R * kda::TR_H_ELEMS * 2);
    L.vn = off;
    off = align256(off + (size_t)R * kda::TR_VN_ELEMS * 2);
    L.dh = off;
    off = align256(off + (size_t)R * kda::TR_H_ELEMS * 2);
    L.dvn = off;
    off = align256(off + (size_t)R * kda::TR_VN_ELEMS * 2);
    L.part = off;
    off = align256(off + (size_t)R * kda::PART_STRIDE * 4);
    L.total = off;
    return L;
}

// The state a training forward keeps for its backward (kda_bt16_fwd_save_hip),
// per record slot: the backward record, h, v_new and the gram block.
struct SavedLayout {
    size_t brec, h, vn, la, total;
};

SavedLayout saved_layout(int64_t R) {
    SavedLayout L;
    size_t off = 0;
    L.brec = off;
    off = align256(off + (size_t)R * kda::REC_BYTES);
    L.h = off;
    off = align256(off + (size_t)R * kda::TR_H_ELEMS * 2);
    L.vn = off;
    off = align256(off + (size_t)R * kda::TR_VN_ELEMS * 2);
    L.la = off;
    off = align256(off + (size_t)R * kda::LA_BYTES);
    L.total = off;
    return L;
}

// The backward's workspace when the state was saved: dh, dv_new and the
// gate partial sums.
struct BwdSavedLayout {
    size_t dh, dvn, part, total;
};

BwdSavedLayout bwd_saved_layout(int64_t R) {
    BwdSavedLayout L;
    size_t off = 0;
    L.dh = off;
    off = align256(off + (size_t)R * kda::TR_H_ELEMS * 2);
    L.dvn = off;
    off = align256(off + (size_t)R * kda::TR_VN_ELEMS * 2);
    L.part = off;
    off = align256(off + (size_t)R * kda::PART_STRIDE * 4);
    L.total = off;
    return L;
}

// Checks of a backward call (both entry points) and its Params, without
// the workspace.
int bwd_params(const KdaBt16BwdArgs* b, Params& p) {
    if (b == nullptr || b->fwd == nullptr) return KDA_BT16_EINVAL;
    const KdaBt16Args* a = b->fwd;
    int rc = check_common(a, p);
    if (rc != KDA_BT16_OK) return rc;
    if (a->flags & KDA_BT16_O_FP32) return KDA_BT16_EUNSUPPORTED;
    const int64_t slots = a->cu_seqlens ? varlen_slots(a) : (int64_t)a->B * chunks_of(a->T);
    if ((int64_t)a->HV * slots > I32_MAX || sequences(a) * a->HV * 8 > I32_MAX ||
        chunks_of(a->T) * kda::REC_BYTES > I32_MAX)
        return KDA_BT16_EUNSUPPORTED;
    p.NS = a->cu_seqlens ? (int)varlen_slots(a) : 0;
    if (!a->q || !a->k || !a->v || !a->g || !a->beta) return KDA_BT16_EINVAL;
    if (p.use_gate && !a->A_log) return KDA_BT16_EINVAL;
    if (a->dbg_Aqk || a->dbg_A_inv || a->dbg_w || a->dbg_u || a->dbg_g) return KDA_BT16_EINVAL;
    if (!b->dout || !b->dq || !b->dk || !b->dv || !b->dg || !b->dbeta) return KDA_BT16_EINVAL;
    if ((b->dA_log || b->ddt_bias) && !p.use_gate) return KDA_BT16_EINVAL;
    if (b->ddt_bias && !a->dt_bias) return KDA_BT16_EINVAL;
    const uintptr_t bsz = a->beta_dtype == KDA_BT16_DTYPE_BF16 ? 2 : 4;
    if (misaligned(a->q, 16) || misaligned(a->k, 16) || misaligned(a->v, 16) ||
        misaligned(a->g, 16) || misaligned(a->beta, bsz) || misaligned(a->dt_bias, 16) ||
        misaligned(a->h0, 16) || misaligned(b->dout, 16) || misaligned(b->dht, 16) ||
        misaligned(b->dq, 16) || misaligned(b->dk, 16) || misaligned(b->dv, 16) ||
        misaligned(b->dg, 16) || misaligned(b->dbeta, bsz) || misaligned(b->dh0, 16) ||
        misaligned(b->dA_log, 4) || misaligned(b->ddt_bias, 4))
        return KDA_BT16_EINVAL;
    p.o = nullptr;
    p.ht = nullptr;
    p.dout = static_cast<const uint16_t*>(b->dout);
    p.dht = b->dht;
    p.dq = static_cast<uint16_t*>(b->dq);
    p.dk = static_cast<uint16_t*>(b->dk);
    p.dv = static_cast<uint16_t*>(b->dv);
    p.dg = b->dg;
    p.dbeta = b->dbeta;
    p.dA_log = b->dA_log;
    p.ddt_bias = b->ddt_bias;
    p.dh0 = b->dh0;
    return KDA_BT16_OK;
}

bool bad_buffer(const void* buf, size_t bytes, size_t need) {
    return buf == nullptr || bytes < need || (reinterpret_cast<uintptr_t>(buf) & 255u) != 0;
}

}  // namespace

extern "C" {

size_t kda_bt16_workspace_bytes(int32_t B, int32_t T, int32_t HV, int32_t K, int32_t V) {
    if (B <= 0 || T <= 0 || HV <= 0 || K != kda::DK || V != kda::DK) return 0;
    return (size_t)B * (size_t)HV * (size_t)chunks_of(T) * (size_t)kda::REC_BYTES;
}

size_t kda_bt16_workspace_bytes_args(const KdaBt16Args* a) {
    if (a == nullptr || a->T <= 0 || a->HV <= 0 || a->K != kda::DK || a->V != kda::DK) return 0;
    if (!a->cu_seqlens) return kda_bt16_workspace_bytes(a->B, a->T, a->HV, a->K, a->V);
    if (a->N <= 0) return 0;
    return (size_t)a->HV * (size_t)varlen_slots(a) * (size_t)kda::REC_BYTES;
}

int kda_bt16_k1_hip(const KdaBt16Args* args, void* stream) {
    Params p;
    int rc = to_params(args, p, true, false);
    if (rc != KDA_BT16_OK) return rc;
    if (kda::launch_k1(p, static_cast<hipStream_t>(stream)) != hipSuccess) return KDA_BT16_ELAUNCH;
    return KDA_BT16_OK;
}

int kda_bt16_k2_hip(const KdaBt16Args* args, void* stream) {
    Params p;
    int rc = to_params(args, p, false, true);
    if (rc != KDA_BT16_OK) return rc;
    if (kda::launch_k2(p, static_cast<hipStream_t>(stream)) != hipSuccess) return KDA_BT16_ELAUNCH;
    return KDA_BT16_OK;
}

int kda_bt16_fwd_hip(const KdaBt16Args* args, void* stream) {
    Params p;
    int rc = to_params_core(args, p, true, true);
    if (rc != KDA_BT16_OK) return rc;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    // The fused forward keeps its records in LDS: no workspace.
    if (kda::fwd_plan(p) == 1) return kda::launch_fused(p, s) == hipSuccess ? KDA_BT16_OK : KDA_BT16_ELAUNCH;
    rc = take_workspace(args, p);
    if (rc != KDA_BT16_OK) return rc;
    if (kda::launch_two_stage(p, s) != hipSuccess) return KDA_BT16_ELAUNCH;
    return KDA_BT16_OK;
}

int kda_bt16_fwd_plan(const KdaBt16Args* args) {
    Params p;
    const int rc = to_params_core(args, p, true, true);
    if (rc != KDA_BT16_OK) return rc;
    return kda::fwd_plan(p);
}

int kda_bt16_fwd_segments(const KdaBt16Args* args) {
    Params p;
    const int rc = to_params_core(args, p, true, true);
    if (rc != KDA_BT16_OK) return rc;
    return kda::fwd_plan(p) == 1 ? 0 : kda::fwd_segments(p);
}

int kda_bt16_fused_aborts(uint32_t* count, int32_t reset) {
    if (count == nullptr) return KDA_BT16_EINVAL;
    return kda::fused_abort_count(count, reset != 0) == hipSuccess ? KDA_BT16_OK : KDA_BT16_ELAUNCH;
}

int kda_bt16_fwd_noalloc_hip(const KdaBt16Args* args, void* stream) {
    Params p;
    int rc = to_params_core(args, p, true, true);
    if (rc != KDA_BT16_OK) return rc;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    // The fused forward keeps its records in LDS: no scratch, any size.
    if (kda::fwd_plan(p) == 1) return kda::launch_fused(p, s) == hipSuccess ? KDA_BT16_OK : KDA_BT16_ELAUNCH;
    // The two stages in as many chunk ranges as the forward takes, or more,
    // shorter ones when that many do not fit the scratch.
    const int64_t cap = (int64_t)KDA_BT16_NOALLOC_MAX_WORKSPACE;
    int nseg = kda::fwd_segments(p);
    const bool fits = nseg == 1 ? kda_bt16_workspace_bytes_args(args) <= (size_t)cap
                                : kda::segment_bytes(p, nseg) <= cap;
    if (!fits) nseg = kda::segments_to_fit(p, cap);
    if (nseg == 0) return KDA_BT16_ESCRATCH;
    rc = scratch_ptr(&p.ws);
    if (rc != KDA_BT16_OK) return rc;
    if (kda::launch_two_stage_in(p, nseg, s) != hipSuccess) return KDA_BT16_ELAUNCH;
    return KDA_BT16_OK;
}

int kda_recurrent_fwd_hip(const KdaBt16Args* args, void* stream) {
    Params p;
    int rc = to_params_recurrent(args, p);
    if (rc != KDA_BT16_OK) return rc;
    if (kda::launch_recurrent(p, static_cast<hipStream_t>(stream)) != hipSuccess)
        return KDA_BT16_ELAUNCH;
    return KDA_BT16_OK;
}

size_t kda_bt16_bwd_workspace_bytes(const KdaBt16Args* a) {
    if (kda_bt16_workspace_bytes_args(a) == 0) return 0;
    return bwd_layout(record_slots(a)).total;
}

int kda_bt16_bwd_hip(const KdaBt16BwdArgs* b, void* stream) {
    Params p;
    int rc = bwd_params(b, p);
    if (rc != KDA_BT16_OK) return rc;
    const BwdLayout L = bwd_layout(record_slots(b->fwd));
    if (bad_buffer(b->workspace, b->workspace_bytes, L.total)) return KDA_BT16_EWORKSPACE;
    uint8_t* ws = static_cast<uint8_t*>(b->workspace);
    p.ws = ws + L.rec;
    p.ws_bwd = ws + L.brec;
    p.la = ws + L.rec + kda::REC_QG;  // the gram blocks in qg's bytes
    p.la_stride = kda::REC_BYTES;
    p.tr_h = reinterpret_cast<uint16_t*>(ws + L.h);
    p.tr_vn = reinterpret_cast<uint16_t*>(ws + L.vn);
    p.tr_dh = reinterpret_cast<uint16_t*>(ws + L.dh);
    p.tr_dvn = reinterpret_cast<uint16_t*>(ws + L.dvn);
    p.tr_part = (b->dA_log || b->ddt_bias) ? reinterpret_cast<float*>(ws + L.part) : nullptr;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (kda::launch_k1_both_records(p, s) != hipSuccess) return KDA_BT16_ELAUNCH;
    if (kda::launch_k2_train(p, s) != hipSuccess) return KDA_BT16_ELAUNCH;
    if (kda::launch_k2_bwd(p, s) != hipSuccess) return KDA_BT16_ELAUNCH;
    if (kda::launch_bwd_chunk(p, s) != hipSuccess) return KDA_BT16_ELAUNCH;
    if (p.tr_part && kda::launch_bwd_gate_reduce(p, s) != hipSuccess) return KDA_BT16_ELAUNCH;
    return KDA_BT16_OK;
}

size_t kda_bt16_saved_bytes(const KdaBt16Args* fwd) {
    if (kda_bt16_workspace_bytes_args(fwd) == 0) return 0;
    return saved_layout(record_slots(fwd)).total;
}

int kda_bt16_fwd_save_hip(const KdaBt16Args* args, void* saved, size_t saved_bytes, void* stream) {
    Params p;
    int rc = to_params(args, p, true, true);
    if (rc != KDA_BT16_OK) return rc;
    if (args->dbg_Aqk || args->dbg_A_inv || args->dbg_w || args->dbg_u || args->dbg_g)
        return KDA_BT16_EINVAL;
    const SavedLayout L = saved_layout(record_slots(args));
    if (bad_buffer(saved, saved_bytes, L.total)) return KDA_BT16_EWORKSPACE;
    uint8_t* sv = static_cast<uint8_t*>(saved);
    p.ws_bwd = sv + L.brec;
    p.tr_h = reinterpret_cast<uint16_t*>(sv + L.h);
    p.tr_vn = reinterpret_cast<uint16_t*>(sv + L.vn);
    p.la = sv + L.la;
    p.la_stride = kda::LA_BYTES;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (kda::launch_fwd_save(p, s) != hipSuccess) return KDA_BT16_ELAUNCH;
    return KDA_BT16_OK;
}

size_t kda_bt16_bwd_saved_workspace_bytes(const KdaBt16Args* fwd) {
    if (kda_bt16_workspace_bytes_args(fwd) == 0) return 0;
    return bwd_saved_layout(record_slots(fwd)).total;
}

int kda_bt16_bwd_saved_hip(const KdaBt16BwdArgs* b, void* saved, size_t saved_bytes, void* stream) {
    Params p;
    int rc = bwd_params(b, p);
    if (rc != KDA_BT16_OK) return rc;
    const int64_t R = record_slots(b->fwd);
    const SavedLayout S = saved_layout(R);
    const BwdSavedLayout L = bwd_saved_layout(R);
    if (bad_buffer(saved, saved_bytes, S.total)) return KDA_BT16_EWORKSPACE;
    if (bad_buffer(b->workspace, b->workspace_bytes, L.total)) return KDA_BT16_EWORKSPACE;
    uint8_t* sv = static_cast<uint8_t*>(saved);
    uint8_t* ws = static_cast<uint8_t*>(b->workspace);
    p.ws = nullptr;
    p.ws_bwd = sv + S.brec;
    p.tr_h = reinterpret_cast<uint16_t*>(sv + S.h);
    p.tr_vn = reinterpret_cast<uint16_t*>(sv + S.vn);
    p.la = sv + S.la;
    p.la_stride = kda::LA_BYTES;
    p.tr_dh = reinterpret_cast<uint16_t*>(ws + L.dh);
    p.tr_dvn = reinterpret_cast<uint16_t*>(ws + L.dvn);
    p.tr_part = (b->dA_log || b->ddt_bias) ? reinterpret_cast<float*>(ws + L.part) : nullptr;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (kda::launch_k1_dout(p, s) != hipSuccess) return KDA_BT16_ELAUNCH;
    if (kda::launch_k2_bwd(p, s) != hipSuccess) return KDA_BT16_ELAUNCH;
    if (kda::launch_bwd_chunk(p, s) != hipSuccess) return KDA_BT16_ELAUNCH;
    if (p.tr_part && kda::launch_bwd_gate_reduce(p, s) != hipSuccess) return KDA_BT16_ELAUNCH;
    return KDA_BT16_OK;
}

const char* kda_bt16_strerror(int code) {
    switch (code) {
        case KDA_BT16_OK: return "ok";
        case KDA_BT16_EINVAL:
            return "invalid argument (null pointer, non-positive size, bad dtype tag, "
                   "misaligned tensor, cu_seqlens with B != 1 or N <= 0, both FUSED_KERNEL and "
                   "TWO_STAGE, or a kernel choice out of range)";
        case KDA_BT16_EUNSUPPORTED:
            return "unsupported geometry (needs K=V=128, HV a multiple of H, T <= 1973776 and "
                   "32-bit grids) or flag";
        case KDA_BT16_EWORKSPACE: return "workspace missing, misaligned or smaller than kda_bt16_workspace_bytes_args()";
        case KDA_BT16_ELAUNCH: return "HIP kernel launch failed";
        case KDA_BT16_EABI: return "abi_version mismatch";
        case KDA_BT16_ERANGE: return "lower_bound must be in (-11, 0) with the in-kernel gate";
        case KDA_BT16_ESCRATCH:
            return "kda_bt16_fwd_noalloc_hip: the geometry needs more records than its static "
                   "scratch holds (KDA_BT16_NOALLOC_MAX_WORKSPACE, 96 MiB), even in chunk ranges "
                   "(packed sequences and debug outputs run in one pass); use kda_bt16_fwd_hip "
                   "with a workspace";
        default: return "unknown error";
    }
}

int kda_bt16_abi_version(void) { return KDA_BT16_ABI_VERSION; }

}  // extern "C"
