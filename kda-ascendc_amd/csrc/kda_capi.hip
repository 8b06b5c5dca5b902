// C ABI of libkda_bt16_hip.so: argument checks, the two stage launches and
// the token recurrence.
// The checks here guard the kernels' indexing assumptions (shapes, pointer
// presence, workspace size); the user-facing validation with the
// reference's messages lives in the Python layer.
#include "../../include/kda_bt16_hip.h"
#include "kda_common.h"

namespace {

using kda::Params;

bool misaligned(const void* p, uintptr_t align) {
    return (reinterpret_cast<uintptr_t>(p) & (align - 1)) != 0;
}

int to_params(const KdaBt16Args* a, Params& p, bool need_inputs, bool need_outputs) {
    if (a == nullptr) return KDA_BT16_EINVAL;
    if (a->abi_version != KDA_BT16_ABI_VERSION) return KDA_BT16_EABI;
    if (a->B <= 0 || a->T <= 0 || a->H <= 0 || a->HV <= 0 || a->K <= 0 || a->V <= 0)
        return KDA_BT16_EINVAL;
    if (a->K != kda::DK || a->V != kda::DK || a->HV != a->H) return KDA_BT16_EUNSUPPORTED;
    if (a->flags & KDA_BT16_O_FP32) return KDA_BT16_EUNSUPPORTED;
    // Grid sizes are 32-bit (B*H*NT work-groups for stage 1, B*H*8 for stage
    // 2), and stage 2 addresses one head's records through a buffer
    // descriptor with a 32-bit size (NT * REC_BYTES bytes).
    const int64_t nt = ((int64_t)a->T + kda::BT - 1) / kda::BT;
    if ((int64_t)a->B * a->H * nt > 0x7fffffffLL || nt * kda::REC_BYTES > 0x7fffffffLL)
        return KDA_BT16_EUNSUPPORTED;
    if ((a->g_dtype != KDA_BT16_DTYPE_F32 && a->g_dtype != KDA_BT16_DTYPE_BF16) ||
        (a->beta_dtype != KDA_BT16_DTYPE_F32 && a->beta_dtype != KDA_BT16_DTYPE_BF16))
        return KDA_BT16_EINVAL;
    const bool use_gate = (a->flags & KDA_BT16_USE_GATE) != 0;
    if (use_gate && !(a->lower_bound > -11.0f && a->lower_bound < 0.0f)) return KDA_BT16_ERANGE;
    if (need_inputs) {
        if (!a->q || !a->k || !a->v || !a->g || !a->beta) return KDA_BT16_EINVAL;
        if (use_gate && !a->A_log) return KDA_BT16_EINVAL;
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
    const size_t need = kda_bt16_workspace_bytes(a->B, a->T, a->H, a->K, a->V);
    if (!a->workspace || a->workspace_bytes < need) return KDA_BT16_EWORKSPACE;
    if ((reinterpret_cast<uintptr_t>(a->workspace) & 255u) != 0) return KDA_BT16_EWORKSPACE;

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
    p.ws = static_cast<uint8_t*>(a->workspace);
    p.dbg_Aqk = static_cast<uint16_t*>(a->dbg_Aqk);
    p.dbg_A_inv = static_cast<uint16_t*>(a->dbg_A_inv);
    p.dbg_w = static_cast<uint16_t*>(a->dbg_w);
    p.dbg_u = static_cast<uint16_t*>(a->dbg_u);
    p.dbg_g = a->dbg_g;
    p.B = a->B;
    p.T = a->T;
    p.H = a->H;
    p.NT = (a->T + kda::BT - 1) / kda::BT;
    p.scale = a->scale;
    p.lower_bound = a->lower_bound;
    p.g_bf16 = a->g_dtype == KDA_BT16_DTYPE_BF16;
    p.beta_bf16 = a->beta_dtype == KDA_BT16_DTYPE_BF16;
    p.use_gate = use_gate;
    p.use_l2norm = (a->flags & KDA_BT16_USE_QK_L2NORM) != 0;
    p.use_beta_sigmoid = (a->flags & KDA_BT16_USE_BETA_SIGMOID) != 0;
    p.h0_v_first = p.ht_v_first = (a->flags & KDA_BT16_STATE_V_FIRST) != 0;
    p.HV = a->H;
    p.o_fp32 = 0;
    return KDA_BT16_OK;
}

// The token recurrence: HV a multiple of H, no workspace, no debug outputs,
// o in bf16 or fp32.
int to_params_recurrent(const KdaBt16Args* a, Params& p) {
    if (a == nullptr) return KDA_BT16_EINVAL;
    if (a->abi_version != KDA_BT16_ABI_VERSION) return KDA_BT16_EABI;
    if (a->B <= 0 || a->T <= 0 || a->H <= 0 || a->HV <= 0 || a->K <= 0 || a->V <= 0)
        return KDA_BT16_EINVAL;
    if (a->K != kda::DK || a->V != kda::DK || a->HV % a->H != 0) return KDA_BT16_EUNSUPPORTED;
    if ((int64_t)a->B * a->HV > 0x7fffffffLL) return KDA_BT16_EUNSUPPORTED;
    if ((a->g_dtype != KDA_BT16_DTYPE_F32 && a->g_dtype != KDA_BT16_DTYPE_BF16) ||
        (a->beta_dtype != KDA_BT16_DTYPE_F32 && a->beta_dtype != KDA_BT16_DTYPE_BF16))
        return KDA_BT16_EINVAL;
    const bool use_gate = (a->flags & KDA_BT16_USE_GATE) != 0;
    if (use_gate && !(a->lower_bound > -11.0f && a->lower_bound < 0.0f)) return KDA_BT16_ERANGE;
    if (!a->q || !a->k || !a->v || !a->g || !a->beta || !a->o) return KDA_BT16_EINVAL;
    if (use_gate && !a->A_log) return KDA_BT16_EINVAL;
    if (a->dbg_Aqk || a->dbg_A_inv || a->dbg_w || a->dbg_u || a->dbg_g) return KDA_BT16_EINVAL;
    // 16-byte state rows; 2-byte q/k/v elements read in pairs.
    if (misaligned(a->q, 4) || misaligned(a->k, 4) || misaligned(a->v, 2) ||
        misaligned(a->g, a->g_dtype == KDA_BT16_DTYPE_BF16 ? 2 : 4) ||
        misaligned(a->beta, a->beta_dtype == KDA_BT16_DTYPE_BF16 ? 2 : 4) ||
        misaligned(a->dt_bias, 4) || misaligned(a->h0, 16) || misaligned(a->ht, 16) ||
        misaligned(a->o, (a->flags & KDA_BT16_O_FP32) ? 4 : 2))
        return KDA_BT16_EINVAL;

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
    p.H = a->H;
    p.HV = a->HV;
    p.scale = a->scale;
    p.lower_bound = a->lower_bound;
    p.g_bf16 = a->g_dtype == KDA_BT16_DTYPE_BF16;
    p.beta_bf16 = a->beta_dtype == KDA_BT16_DTYPE_BF16;
    p.use_gate = use_gate;
    p.use_l2norm = (a->flags & KDA_BT16_USE_QK_L2NORM) != 0;
    p.use_beta_sigmoid = (a->flags & KDA_BT16_USE_BETA_SIGMOID) != 0;
    p.h0_v_first = p.ht_v_first = (a->flags & KDA_BT16_STATE_V_FIRST) != 0;
    p.o_fp32 = (a->flags & KDA_BT16_O_FP32) != 0;
    return KDA_BT16_OK;
}

}  // namespace

extern "C" {

size_t kda_bt16_workspace_bytes(int32_t B, int32_t T, int32_t H, int32_t K, int32_t V) {
    if (B <= 0 || T <= 0 || H <= 0 || K != kda::DK || V != kda::DK) return 0;
    const size_t nt = (size_t)(T + kda::BT - 1) / kda::BT;
    return (size_t)B * (size_t)H * nt * (size_t)kda::REC_BYTES;
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
    int rc = to_params(args, p, true, true);
    if (rc != KDA_BT16_OK) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (kda::launch_k1(p, s) != hipSuccess) return KDA_BT16_ELAUNCH;
    if (kda::launch_k2(p, s) != hipSuccess) return KDA_BT16_ELAUNCH;
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

const char* kda_bt16_strerror(int code) {
    switch (code) {
        case KDA_BT16_OK: return "ok";
        case KDA_BT16_EINVAL: return "invalid argument (null pointer, non-positive size or bad dtype tag)";
        case KDA_BT16_EUNSUPPORTED:
            return "unsupported geometry (needs K=V=128, HV == H (HV a multiple of H for the "
                   "recurrence) and T <= 1973776) or flag";
        case KDA_BT16_EWORKSPACE: return "workspace missing, misaligned or smaller than kda_bt16_workspace_bytes()";
        case KDA_BT16_ELAUNCH: return "HIP kernel launch failed";
        case KDA_BT16_EABI: return "abi_version mismatch";
        case KDA_BT16_ERANGE: return "lower_bound must be in (-11, 0) with the in-kernel gate";
        default: return "unknown error";
    }
}

int kda_bt16_abi_version(void) { return KDA_BT16_ABI_VERSION; }

}  // extern "C"
