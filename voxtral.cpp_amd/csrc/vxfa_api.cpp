// vxfa_api.cpp — the C ABI of include/vxfa.h: contract validation (the
// supports_op analogue), per-stream context with the split-KV workspace, and
// dispatch to the gfx950 kernels.
//
// The validation rules restate the asserts ggml_flash_attn_ext makes when it
// builds the node (q/k/v/mask shapes, GQA and batch broadcast divisibility)
// and the CPU kernel's layout requirements (contiguous rows, dst contiguous
// in the permuted order), as used at src/voxtral.cpp:1611 and :1802.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>
#include <new>

#include "../../include/vxfa.h"
#include "fa_common.h"

// Device workspace of a context, allocated once by vxfa_ctx_create (no call
// allocates, frees or synchronises): the split-KV partial records and f16
// staging for F32 K/V of prefill calls.
constexpr size_t kRecordBytes = (size_t)8 << 20;        // e.g. 256 (batch, kv head) pairs x 8 splits, or 8 x 64
constexpr size_t kStageBytes = (size_t)32 << 20;        // F32 K and V of 8192 rows x 1024 as f16

// Launch-shape overrides for tuning sweeps (VXFA_DECODE_SPLIT,
// VXFA_PREFILL_WAVES, VXFA_PREFILL_PP, VXFA_PREFILL_PAIR), read from the
// environment; 0 = heuristic.
struct Tuning {
    int split_override = 0;
    int waves_override = 0;
    // VXFA_PREFILL_PP=0 routes hd 64 prefill to the general kernel
    bool pp_enabled = true;
    // VXFA_PREFILL_PAIR=0 routes short masked hd 128 prefill to the general kernel
    bool pair_enabled = true;
    // VXFA_PAIR_INTERVALS=0: with F32 K/V and a mask tensor the short masked
    // prefill classifies its blocks from the mask itself rather than from the
    // intervals a pre-pass finds in the staging launch
    bool pair_intervals = true;
    void read_env() {
        if (const char* e = getenv("VXFA_DECODE_SPLIT")) split_override = atoi(e);
        if (const char* e = getenv("VXFA_PREFILL_WAVES")) waves_override = atoi(e);
        if (const char* e = getenv("VXFA_PREFILL_PP")) pp_enabled = atoi(e) != 0;
        if (const char* e = getenv("VXFA_PREFILL_PAIR")) pair_enabled = atoi(e) != 0;
        if (const char* e = getenv("VXFA_PAIR_INTERVALS")) pair_intervals = atoi(e) != 0;
    }
};

// Where one call may put its device scratch (split-KV partial records of a
// decode call, f16 staging of F32 K/V of a prefill call) and its error
// message: a context's workspace, or the library's static scratch array.
struct Workspace {
    int device;
    float* rec;           // split-KV partial records
    size_t rec_bytes;
    _Float16* stage;      // f16 staging of F32 K/V (prefill)
    size_t stage_bytes;
    char* err;            // message of the last failure
    size_t err_len;
    Tuning tune;
};

struct vxfa_ctx {
    int device = 0;
    char* ws = nullptr;           // one device allocation holding both regions
    float* rec = nullptr;         // kRecordBytes of partial records
    _Float16* stage = nullptr;    // kStageBytes of f16 K/V staging
    char last_error[256] = {0};
    Tuning tune;                  // read once when the context is created
    Workspace view() {
        return Workspace{device, rec, kRecordBytes, stage, kStageBytes, last_error, sizeof(last_error), tune};
    }
};

// Device scratch of vxfa_flash_attn_ext_noalloc: a file-scope array in the
// library's code object (each GPU holds its own copy until the process
// ends), used for the same purposes as a context's workspace. Its device
// address is looked up once per device (hipGetSymbolAddress) and kept; host
// code uses only that address, never the array's name, which on the host is
// a stand-in symbol, not device memory. Every call on one GPU shares the
// array: calls that overlap on one GPU (two streams, two threads) race.
constexpr size_t kScratchBytes = (size_t)8 << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices] = {nullptr};
static thread_local char t_noalloc_err[256] = {0};   // message of this thread's last failing no-alloc call

namespace {

constexpr int kVersion = 1 * 10000 + 1 * 100 + 0;
constexpr int kMaskedSplitCap = 32;

void set_err(Workspace& w, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(w.err, w.err_len, fmt, ap);
    va_end(ap);
}

int elt_size(int32_t t) { return t == VXFA_TYPE_F32 ? 4 : (t == VXFA_TYPE_F16 ? 2 : 0); }

bool aligned16(const void* p, size_t off) { return ((reinterpret_cast<uintptr_t>(p) + off) & 15u) == 0; }

// Returns VXFA_OK / VXFA_INVALID_ARG / VXFA_UNSUPPORTED and a reason.
int check(const vxfa_tensor* q, const vxfa_tensor* k, const vxfa_tensor* v, const vxfa_tensor* mask,
          const vxfa_tensor* dst, float scale, float max_bias, float softcap, const char** why) {
    *why = "";
    if (!q || !k || !v || !dst) { *why = "q, k, v and dst are required"; return VXFA_INVALID_ARG; }
    const vxfa_tensor* all[5] = {q, k, v, dst, mask};
    for (int i = 0; i < 5; ++i) {
        if (!all[i]) continue;
        if (!elt_size(all[i]->type)) { *why = "unknown tensor type"; return VXFA_INVALID_ARG; }
        for (int d = 0; d < 4; ++d)
            if (all[i]->ne[d] < 0) { *why = "negative ne"; return VXFA_INVALID_ARG; }
    }
    // ggml_flash_attn_ext node construction rules
    if (q->ne[0] != k->ne[0]) { *why = "q->ne[0] != k->ne[0]"; return VXFA_INVALID_ARG; }
    if (k->ne[1] != v->ne[1]) { *why = "k->ne[1] != v->ne[1]"; return VXFA_INVALID_ARG; }
    if (k->ne[2] != v->ne[2] || k->ne[3] != v->ne[3]) { *why = "k/v head or batch mismatch"; return VXFA_INVALID_ARG; }
    if (k->ne[2] == 0 || k->ne[3] == 0) { *why = "k has no heads or batches"; return VXFA_INVALID_ARG; }
    if (q->ne[2] % k->ne[2]) { *why = "q heads not a multiple of kv heads"; return VXFA_INVALID_ARG; }
    if (q->ne[3] % k->ne[3]) { *why = "q batch not a multiple of kv batch"; return VXFA_INVALID_ARG; }
    if (mask) {
        if (mask->ne[0] != k->ne[1]) { *why = "mask->ne[0] != n_kv"; return VXFA_INVALID_ARG; }
        if (mask->ne[1] < q->ne[1]) { *why = "mask has fewer rows than q"; return VXFA_INVALID_ARG; }
        if (mask->ne[2] == 0 || mask->ne[3] == 0) { *why = "mask has no planes"; return VXFA_INVALID_ARG; }
        if (q->ne[2] % mask->ne[2] || q->ne[3] % mask->ne[3]) { *why = "mask does not broadcast over q"; return VXFA_INVALID_ARG; }
        if (mask->nb[0] != (size_t)elt_size(mask->type)) { *why = "mask rows not contiguous"; return VXFA_INVALID_ARG; }
    }
    if (dst->ne[0] != v->ne[0] || dst->ne[1] != q->ne[2] || dst->ne[2] != q->ne[1] || dst->ne[3] != q->ne[3]) {
        *why = "dst shape must be [Dv, Hq, Nq, B]";
        return VXFA_INVALID_ARG;
    }
    if (q->nb[0] != (size_t)elt_size(q->type) || k->nb[0] != (size_t)elt_size(k->type) ||
        v->nb[0] != (size_t)elt_size(v->type)) {
        *why = "q/k/v rows must be contiguous";
        return VXFA_INVALID_ARG;
    }
    // what this path implements
    // K/V: f16 (the configured cache) or F32 (the reference's own cache,
    // src/voxtral.cpp:1126-1136, and the encoder's mul_mat outputs, :1581-1605)
    if (k->type != v->type) { *why = "k and v must have one type"; return VXFA_UNSUPPORTED; }
    if (mask && mask->type != VXFA_TYPE_F16) { *why = "mask must be F16"; return VXFA_UNSUPPORTED; }
    if (dst->type != VXFA_TYPE_F32) { *why = "dst must be F32"; return VXFA_UNSUPPORTED; }
    if (dst->nb[0] != 4 || dst->nb[1] != 4 * (size_t)dst->ne[0] || dst->nb[2] != dst->nb[1] * (size_t)dst->ne[1] ||
        dst->nb[3] != dst->nb[2] * (size_t)dst->ne[2]) {
        *why = "dst must be contiguous";
        return VXFA_UNSUPPORTED;
    }
    if (k->ne[0] != v->ne[0]) { *why = "Dk != Dv"; return VXFA_UNSUPPORTED; }
    if (k->ne[0] != 64 && k->ne[0] != 128) { *why = "head dim must be 64 or 128"; return VXFA_UNSUPPORTED; }
    if (max_bias != 0.0f) { *why = "max_bias (ALiBi) not implemented"; return VXFA_UNSUPPORTED; }
    if (softcap != 0.0f) { *why = "logit_softcap not implemented"; return VXFA_UNSUPPORTED; }
    if (!isfinite(scale)) { *why = "scale must be finite"; return VXFA_UNSUPPORTED; }
    const int64_t lim = 0x7fffffff;
    if (q->ne[1] > lim || k->ne[1] > lim || q->ne[2] > 65535 || q->ne[3] > 65535) {
        *why = "sizes beyond the launch limits";
        return VXFA_UNSUPPORTED;
    }
    // the prefill kernel addresses up to 256 K/V rows from one base with
    // 32-bit offsets
    if (k->nb[1] >= ((size_t)1 << 23) || v->nb[1] >= ((size_t)1 << 23)) {
        *why = "k/v row stride must be below 8 MiB";
        return VXFA_UNSUPPORTED;
    }
    // 128-bit loads: q/k/v rows and dst rows must be 16-byte aligned
    const vxfa_tensor* vec[4] = {q, k, v, dst};
    for (int i = 0; i < 4; ++i) {
        if (!aligned16(vec[i]->data, 0) || (vec[i]->nb[1] & 15) || (vec[i]->nb[2] & 15) || (vec[i]->nb[3] & 15)) {
            *why = "q/k/v/dst data and strides must be 16-byte aligned";
            return VXFA_UNSUPPORTED;
        }
    }
    if (mask && ((reinterpret_cast<uintptr_t>(mask->data) & 1u) || (mask->nb[1] & 1) || (mask->nb[2] & 1) ||
                 (mask->nb[3] & 1))) {
        *why = "mask must be 2-byte aligned";
        return VXFA_UNSUPPORTED;
    }
    return VXFA_OK;
}

// New K/V rows for an append: F32 [Hkv * D, n_new, 1, Bk] with contiguous
// 16-byte-aligned rows, going to the last n_new rows of the F16 cache views
// k, v [D, n_kv, Hkv, Bk] (checked by check()).
int check_append(const vxfa_tensor* k, const vxfa_tensor* v, const vxfa_tensor* kn, const vxfa_tensor* vn,
                 const char** why) {
    if (!kn || !vn) { *why = "k_new and v_new are required"; return VXFA_INVALID_ARG; }
    const vxfa_tensor* nw[2] = {kn, vn};
    const vxfa_tensor* cache[2] = {k, v};
    for (int i = 0; i < 2; ++i) {
        const vxfa_tensor* t = nw[i];
        for (int d = 0; d < 4; ++d)
            if (t->ne[d] < 0) { *why = "negative ne"; return VXFA_INVALID_ARG; }
        if (t->ne[0] != cache[i]->ne[0] * cache[i]->ne[2]) { *why = "new rows must hold Hkv * D elements"; return VXFA_INVALID_ARG; }
        if (t->ne[1] > cache[i]->ne[1]) { *why = "more new rows than cache rows"; return VXFA_INVALID_ARG; }
        if (t->ne[2] != 1 || t->ne[3] != cache[i]->ne[3]) { *why = "new rows must be [Hkv*D, n, 1, Bk]"; return VXFA_INVALID_ARG; }
        if (t->type != VXFA_TYPE_F32) { *why = "new rows must be F32"; return VXFA_UNSUPPORTED; }
        if (t->nb[0] != 4 || !aligned16(t->data, 0) || (t->nb[1] & 15) || (t->nb[3] & 15)) {
            *why = "new rows must be contiguous and 16-byte aligned";
            return VXFA_UNSUPPORTED;
        }
        if (cache[i]->type != VXFA_TYPE_F16) { *why = "the cache must be F16"; return VXFA_UNSUPPORTED; }
        if (cache[i]->ne[0] % 8 || cache[i]->nb[0] != 2 || !aligned16(cache[i]->data, 0) || (cache[i]->nb[1] & 15) ||
            (cache[i]->nb[2] & 15) || (cache[i]->nb[3] & 15)) {
            *why = "cache rows must be contiguous and 16-byte aligned";
            return VXFA_UNSUPPORTED;
        }
    }
    if (kn->ne[1] != vn->ne[1]) { *why = "k_new and v_new row counts differ"; return VXFA_INVALID_ARG; }
    if (k->ne[1] != v->ne[1] || k->ne[2] != v->ne[2] || k->ne[3] != v->ne[3] || k->ne[0] != v->ne[0]) {
        *why = "k and v cache views differ";
        return VXFA_INVALID_ARG;
    }
    if (kn->ne[1] > 0x7fffffff || k->ne[3] > 65535) { *why = "sizes beyond the launch limits"; return VXFA_UNSUPPORTED; }
    return VXFA_OK;
}

vxfa::AppendArgs append_args(const vxfa_tensor* k, const vxfa_tensor* v, const vxfa_tensor* kn,
                             const vxfa_tensor* vn) {
    vxfa::AppendArgs a;
    memset(&a, 0, sizeof(a));
    a.k_new = static_cast<const float*>(kn->data);
    a.v_new = static_cast<const float*>(vn->data);
    a.kn_nb1 = (int64_t)kn->nb[1]; a.kn_nb3 = (int64_t)kn->nb[3];
    a.vn_nb1 = (int64_t)vn->nb[1]; a.vn_nb3 = (int64_t)vn->nb[3];
    a.k = static_cast<_Float16*>(k->data);
    a.v = static_cast<_Float16*>(v->data);
    a.k_nb1 = (int64_t)k->nb[1]; a.k_nb2 = (int64_t)k->nb[2]; a.k_nb3 = (int64_t)k->nb[3];
    a.v_nb1 = (int64_t)v->nb[1]; a.v_nb2 = (int64_t)v->nb[2]; a.v_nb3 = (int64_t)v->nb[3];
    a.d = (int32_t)k->ne[0];
    a.hkv = (int32_t)k->ne[2];
    a.n_new = (int32_t)kn->ne[1];
    a.pos0 = (int32_t)(k->ne[1] - kn->ne[1]);
    a.bk = (int32_t)k->ne[3];
    return a;
}

// Workgroups per (batch, kv head) for the decode split kernel: 2048
// wavefronts in all (8 per CU), at least four tiles of live positions per
// workgroup (one 16 KB tile for each of its four wavefronts, and no
// wavefront with a second: 128 positions of an f16 cache, 64 of an F32 one),
// and at most kDecodeMaxSplit so the merge stays short.
// Measured in graph replays at 8 kv heads (split + combine, us per layer):
// n_kv 1024 8.30 with 8 splits against 8.39 with 16; 2048 8.67 (16) against
// 8.77 (32); 3000 8.83 (24) against 11.12 (48); 4096 9.25 (32) against
// 11.30 (64); 8192 12.25 (64) against 12.99 (32). With a mask tensor every
// split workgroup scans the whole mask row, so the caller caps the count
// (measured on a 2048 window of a 16K cache).
// Tile size: *t16 is set when f16 tiles of 32 positions would leave fewer
// workgroups than the target (short spans: n_kv 1024, a 2048 window); the
// tiles then hold 16 positions, as F32 tiles do, and the split count doubles
// for the same span (n_kv 1024 7.01 -> 6.55 us per layer, a 2048-row ring
// with append 8.61 -> 7.67; at n_kv 8192, where tiles of 32 already fill the
// grid, tiles of 16 measured slower, 10.96 -> 12.07, and tiles of 8 on short
// spans gained nothing at 1024 and lost 0.4-0.8 us on the 2048 window).
int choose_split(int64_t pairs, int64_t nkv, bool kv_f32, bool* t16) {
    const int64_t target = 2048 / vxfa::kDecodeWaves;
    int64_t s = (target + pairs - 1) / pairs;
    int64_t per = (int64_t)vxfa::kDecodeWaves * (kv_f32 ? 16 : 32);   // one tile per wavefront
    int64_t by_len = (nkv + per - 1) / per;
    *t16 = false;
    if (!kv_f32 && by_len < s) {
        *t16 = true;
        per = (int64_t)vxfa::kDecodeWaves * 16;
        by_len = (nkv + per - 1) / per;
    }
    if (s > by_len) s = by_len;
    if (s > vxfa::kDecodeMaxSplit) s = vxfa::kDecodeMaxSplit;
    if (s < 1) s = 1;
    return (int)s;
}

// The split count a workspace of rec_bytes can hold: pairs * S records of
// rec_floats each (else fewer splits, down to none).
int fit_split(int S, int64_t pairs, int rec_floats, size_t rec_bytes) {
    if (S <= 1) return 1;
    const int64_t cap = (int64_t)(rec_bytes / sizeof(float)) / (pairs * rec_floats);
    if (cap < 2) return 1;
    return S < cap ? S : (int)cap;
}

}  // namespace

extern "C" {

vxfa_ctx* vxfa_ctx_create(int device) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return nullptr;
    vxfa_ctx* c = new (std::nothrow) vxfa_ctx();
    if (!c) return nullptr;
    c->device = device;
    c->tune.read_env();
    int prev = 0;
    (void)hipGetDevice(&prev);
    const bool ok = hipSetDevice(device) == hipSuccess && hipMalloc(&c->ws, kRecordBytes + kStageBytes) == hipSuccess;
    (void)hipSetDevice(prev);
    if (!ok) {
        delete c;
        return nullptr;
    }
    c->rec = reinterpret_cast<float*>(c->ws);
    c->stage = reinterpret_cast<_Float16*>(c->ws + kRecordBytes);
    return c;
}

void vxfa_ctx_destroy(vxfa_ctx* c) {
    if (!c) return;
    int prev = 0;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(c->device);
    if (c->ws) {
        (void)hipDeviceSynchronize();
        (void)hipFree(c->ws);
    }
    (void)hipSetDevice(prev);
    delete c;
}

int vxfa_supports(const vxfa_tensor* q, const vxfa_tensor* k, const vxfa_tensor* v, const vxfa_tensor* mask,
                  const vxfa_tensor* dst, float scale, float max_bias, float logit_softcap) {
    const char* why = nullptr;
    return check(q, k, v, mask, dst, scale, max_bias, logit_softcap, &why);
}

const char* vxfa_status_str(int s) {
    switch (s) {
        case VXFA_OK: return "ok";
        case VXFA_UNSUPPORTED: return "unsupported";
        case VXFA_INVALID_ARG: return "invalid argument";
        case VXFA_NO_WORKSPACE: return "no workspace";
        case VXFA_HIP_ERROR: return "hip error";
        default: return "unknown status";
    }
}

const char* vxfa_last_error(const vxfa_ctx* c) { return c ? c->last_error : t_noalloc_err; }

int vxfa_version(void) { return kVersion; }

}  // extern "C"

namespace {

// The op, with either a mask tensor (`mask`), an implicit causal / window mask
// (`im`, kind VXFA_MASK_CAUSAL) or neither; never both (the entry points
// enforce it).
int run(Workspace& w, const vxfa_tensor* q, const vxfa_tensor* k, const vxfa_tensor* v, const vxfa_tensor* mask,
        const vxfa_mask_desc* im, vxfa_tensor* dst, float scale, float max_bias, float logit_softcap, void* stream,
        const vxfa_tensor* k_new = nullptr, const vxfa_tensor* v_new = nullptr, const vxfa_ring* ring = nullptr,
        const vxfa_rope* rope = nullptr) {
    w.err[0] = 0;
    const char* why = nullptr;
    int rc = check(q, k, v, mask, dst, scale, max_bias, logit_softcap, &why);
    if (rc == VXFA_OK && k_new) rc = check_append(k, v, k_new, v_new, &why);
    if (rc == VXFA_OK && rope) {
        if (!rope->positions || !k_new) {
            why = "rope: positions and the new K/V rows are required";
            rc = VXFA_INVALID_ARG;
        } else if (k_new->ne[1] != q->ne[1] || q->ne[3] != k->ne[3]) {
            why = "rope: the new rows are the query tokens (n_new = Nq, one kv batch per q batch)";
            rc = VXFA_INVALID_ARG;
        } else if (rope->n_dims <= 0 || rope->n_dims % 2 || rope->n_dims > q->ne[0]) {
            why = "rope: n_dims must be even and at most the head dim";
            rc = VXFA_INVALID_ARG;
        } else if (rope->mode != 0 || rope->freq_scale != 1.0f || !(rope->freq_base > 0.0f) ||
                   q->type != VXFA_TYPE_F32) {
            why = "rope: mode 0, freq_scale 1, freq_base > 0 and F32 q only";
            rc = VXFA_UNSUPPORTED;
        }
    }
    if (rc == VXFA_OK && ring) {
        const int64_t G = q->ne[2] / k->ne[2];
        if (ring->start < 0 || ring->start >= k->ne[1] || ring->n_kv < 0 || ring->n_kv > k->ne[1]) {
            why = "ring: need 0 <= start < capacity and 0 <= n_kv <= capacity";
            rc = VXFA_INVALID_ARG;
        } else if (k_new && k_new->ne[1] > ring->n_kv) {
            why = "ring: more new rows than rows in use";
            rc = VXFA_INVALID_ARG;
        } else if (q->ne[1] != 1 || !(G == 1 || G == 2 || G == 4) || mask || (k_new && k_new->ne[1] != 1)) {
            why = "ring: single-token decode (GQA group 1, 2 or 4) without a mask, at most one new row";
            rc = VXFA_UNSUPPORTED;
        } else if (k->type != VXFA_TYPE_F16) {
            why = "ring: f16 cache only";
            rc = VXFA_UNSUPPORTED;
        } else if (k->ne[1] >= (1 << 24) ||
                   (int64_t)k->ne[1] * (int64_t)(k->nb[1] > v->nb[1] ? k->nb[1] : v->nb[1]) >= ((int64_t)1 << 31)) {
            // the decode kernel reads a ring's rows by 32-bit offsets from its start
            why = "ring: capacity must be below 2^24 rows and 2 GiB per head slice";
            rc = VXFA_UNSUPPORTED;
        }
    }
    if (rc != VXFA_OK) {
        set_err(w, "%s", why);
        return rc;
    }
    const bool append = k_new != nullptr && k_new->ne[1] > 0;
    const bool implicit = im != nullptr && im->kind == VXFA_MASK_CAUSAL;
    const int64_t D = q->ne[0], Nq = q->ne[1], Hq = q->ne[2], B = q->ne[3];
    const int64_t Nkv = ring ? ring->n_kv : k->ne[1], Hkv = k->ne[2];
    const int64_t Gq = Hq / Hkv;
    // a single new row of a decode step is fused into the split kernel
    const bool fuse_append = append && Nq == 1 && k_new->ne[1] == 1 && (Gq == 1 || Gq == 2 || Gq == 4) &&
                             Nq * Hq * B > 0;

    hipError_t e = hipSetDevice(w.device);
    if (e != hipSuccess) { set_err(w, "hipSetDevice: %s", hipGetErrorString(e)); return VXFA_HIP_ERROR; }
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    // rotary embedding: ggml's theta scale, computed as ggml_rope_ext's CPU path does
    const float rope_ts = rope ? powf(rope->freq_base, -2.0f / (float)rope->n_dims) : 0.0f;
    if (append && !fuse_append) {
        vxfa::AppendArgs ap = append_args(k, v, k_new, v_new);
        if (rope) {
            ap.rope_pos = rope->positions;
            ap.rope_ts = rope_ts;
            ap.rope_dims = rope->n_dims;
        }
        e = vxfa::launch_kv_append(ap, st);
        if (e != hipSuccess) { set_err(w, "kv append: %s", hipGetErrorString(e)); return VXFA_HIP_ERROR; }
    }
    if (Nq * Hq * B == 0) return VXFA_OK;

    if (Nkv == 0) {
        e = vxfa::launch_zero(static_cast<float*>(dst->data), Nq * Hq * B * D, st);
        if (e != hipSuccess) { set_err(w, "zero fill: %s", hipGetErrorString(e)); return VXFA_HIP_ERROR; }
        return VXFA_OK;
    }

    vxfa::AttnArgs a;
    memset(&a, 0, sizeof(a));
    a.q = q->data;
    a.k = static_cast<const _Float16*>(k->data);
    a.v = static_cast<const _Float16*>(v->data);
    a.mask = mask ? static_cast<const uint16_t*>(mask->data) : nullptr;
    a.dst = static_cast<float*>(dst->data);
    a.q_nb1 = (int64_t)q->nb[1]; a.q_nb2 = (int64_t)q->nb[2]; a.q_nb3 = (int64_t)q->nb[3];
    a.k_nb1 = (int64_t)k->nb[1]; a.k_nb2 = (int64_t)k->nb[2]; a.k_nb3 = (int64_t)k->nb[3];
    a.v_nb1 = (int64_t)v->nb[1]; a.v_nb2 = (int64_t)v->nb[2]; a.v_nb3 = (int64_t)v->nb[3];
    if (mask) { a.m_nb1 = (int64_t)mask->nb[1]; a.m_nb2 = (int64_t)mask->nb[2]; a.m_nb3 = (int64_t)mask->nb[3]; }
    a.nq = (int32_t)Nq; a.nkv = (int32_t)Nkv; a.hq = (int32_t)Hq; a.hkv = (int32_t)Hkv;
    a.b = (int32_t)B; a.bk = (int32_t)k->ne[3];
    a.hm = mask ? (int32_t)mask->ne[2] : 1;
    a.bm = mask ? (int32_t)mask->ne[3] : 1;
    a.q_f16 = q->type == VXFA_TYPE_F16;
    a.kv_f32 = k->type == VXFA_TYPE_F32;
    a.mask_vec = mask && aligned16(mask->data, 0) && !(mask->nb[1] & 15) && !(mask->nb[2] & 15) &&
                 !(mask->nb[3] & 15);
    a.scale_log2 = scale * vxfa::kLog2e;
    a.kv_lo = 0;
    a.kv_hi = (int32_t)Nkv;
    if (ring) {
        a.ring_start = (int32_t)ring->start;
        a.ring_cap = (int32_t)k->ne[1];
    }
    if (rope) {
        a.rope_pos = rope->positions;
        a.rope_ts = rope_ts;
        a.rope_dims = rope->n_dims;
    }
    if (fuse_append) {
        a.append = 1;
        a.k_new = static_cast<const float*>(k_new->data);
        a.v_new = static_cast<const float*>(v_new->data);
        a.kn_nb3 = (int64_t)k_new->nb[3];
        a.vn_nb3 = (int64_t)v_new->nb[3];
    }
    if (implicit) {
        a.im_causal = 1;
        a.im_window = im->window;
        a.im_offset = im->offset;
    }

    const int64_t G = Hq / Hkv;
    if (Nq == 1 && (G == 1 || G == 2 || G == 4)) {
        if (implicit) {
            // the one query row attends [offset - W + 1, offset], clipped to [0, n_kv)
            int64_t lo = im->window > 0 ? im->offset - im->window + 1 : 0;
            int64_t hi = im->offset + 1;
            lo = lo < 0 ? 0 : lo;
            hi = hi > Nkv ? Nkv : hi;
            if (hi <= lo) lo = hi = 0;
            a.kv_lo = (int32_t)lo;
            a.kv_hi = (int32_t)hi;
            a.im_causal = 0;   // the range is all the decode kernel needs
        }
        bool t16 = false;
        int S = choose_split(B * Hkv, a.kv_hi - a.kv_lo, a.kv_f32 != 0, &t16);
        // one mask row (a sliding window over a longer cache): the live span,
        // which sets the tiles per split, is found by the kernel; tiles of 16
        // keep every wavefront busy on a window's share (2048 of 16384 rows in
        // 32 splits: 10.29 -> 9.83 us)
        if (mask && B == 1 && !a.kv_f32) t16 = true;
        if (mask && B > 1) {
            // streams of ragged lengths (a mask row each): the longest sets the
            // time, so split every stream finer, about 2048 workgroups in all
            const int64_t s2 = (2048 + B * Hkv - 1) / (B * Hkv);
            if (s2 > S) S = (int)(s2 < (Nkv + 63) / 64 ? s2 : (Nkv + 63) / 64);
        }
        if (mask && S > kMaskedSplitCap) S = kMaskedSplitCap;
        if (w.tune.split_override > 0) S = w.tune.split_override;
        if (S > vxfa::kDecodeMaxSplit) S = vxfa::kDecodeMaxSplit;
        S = fit_split(S, B * Hkv, vxfa::dec_record_floats((int)D, (int)G), w.rec_bytes);
        a.n_split = S;
        a.dec_t16 = t16 ? 1 : 0;
        a.ws = w.rec;
        e = vxfa::launch_decode(a, (int)D, (int)G, st);
    } else {
        size_t staged = 0;   // bytes of the staging area this call fills
        vxfa::StageReq stage;
        if (a.kv_f32) {
            // F32 K/V (the reference's own cache and encoder K/V): an f16 copy
            // in the context's staging area, [Bk][Nkv][Hkv][D], read by the
            // prefill kernels like any f16 view (their tiles reach LDS by
            // direct global-to-LDS copies, which cannot convert); launched
            // below, with the kernel that reads it
            const int64_t Bk = k->ne[3];
            const int64_t per = Bk * Nkv * Hkv * D;
            if ((size_t)(2 * per) * sizeof(_Float16) > w.stage_bytes) {
                set_err(w, "F32 K/V staging needs %lld bytes; the workspace holds %zu",
                        (long long)(2 * per * (int64_t)sizeof(_Float16)), w.stage_bytes);
                return VXFA_NO_WORKSPACE;
            }
            _Float16* sk = w.stage;
            _Float16* sv = w.stage + per;
            stage = vxfa::StageReq{static_cast<const float*>(k->data), (int64_t)k->nb[1], (int64_t)k->nb[2],
                                   (int64_t)k->nb[3], static_cast<const float*>(v->data), (int64_t)v->nb[1],
                                   (int64_t)v->nb[2], (int64_t)v->nb[3], (int)D, (int)Nkv, (int)Hkv, (int)Bk, sk,
                                   sv};
            staged = (size_t)(2 * per) * sizeof(_Float16);
            a.k = sk;
            a.v = sv;
            a.k_nb1 = a.v_nb1 = Hkv * D * 2;
            a.k_nb2 = a.v_nb2 = D * 2;
            a.k_nb3 = a.v_nb3 = Nkv * Hkv * D * 2;
            a.kv_f32 = 0;
        }
        // a mask tensor with a pre-pass (the pipelined hd 64 kernel; the short
        // masked prefill when F32 K/V are staged): the live interval of each
        // mask row (8 bytes a row) in the records region, unused by a prefill
        // call; where records and staging share one area (the no-alloc
        // scratch), after the staged K/V
        int2* mrows = nullptr;
        if (mask) {
            const size_t off = w.rec == reinterpret_cast<float*>(w.stage) ? (staged + 255) & ~(size_t)255 : 0;
            const size_t need = (size_t)(Nq * a.hm * a.bm) * sizeof(int2);
            if (off + need <= w.rec_bytes) mrows = reinterpret_cast<int2*>(reinterpret_cast<char*>(w.rec) + off);
        }
        const bool pp_mask_fits = mrows != nullptr;
        if (D == 64 && (!mask || pp_mask_fits) && !rope && scale != 0.0f && w.tune.pp_enabled) {
            a.mask_rows = mrows;
            // (scale 0 goes to the general kernel: the pipelined one folds the
            // scale into the exponent and scores the partial block's dead rows -inf)
            // encoder prefill: the software-pipelined hd 64 kernel, also under
            // an implicit causal / window mask or a mask tensor (the realtime
            // encoder's window); it launches the F32 staging itself, in the mask
            // pre-pass's launch when there is one
            e = vxfa::launch_prefill64_pp(a, staged ? &stage : nullptr, st);
        } else {
            const bool pair = D == 128 && (mask || implicit) && Nkv <= 512 && w.tune.pair_enabled &&
                              vxfa::prefill_pair_fits(a);
            if (pair && staged && mask && mrows && w.tune.pair_intervals) {
                // the decoder prefill as voxtral calls it (F32 cache, F16 mask):
                // the staging launch also finds the mask rows' intervals, from
                // which the short masked prefill takes its block classes
                a.mask_rows = mrows;
                e = vxfa::launch_mask_prep(a, &stage, st);
                if (e != hipSuccess) { set_err(w, "F32 K/V staging: %s", hipGetErrorString(e)); return VXFA_HIP_ERROR; }
                staged = 0;   // (done in that launch)
            }
            if (staged) {
                e = vxfa::launch_to_f16_kv(stage, st);
                if (e != hipSuccess) { set_err(w, "F32 K/V staging: %s", hipGetErrorString(e)); return VXFA_HIP_ERROR; }
            }
            if (pair) {
                // short masked prefill (voxtral's decoder prefill): paired query
                // tiles, every live block on its own wavefront
                e = vxfa::launch_prefill_pair(a, st);
            } else {
                // query-row wavefronts per workgroup (each with its KV partner
                // wavefronts): 4 shares every staged K/V step among 128 query rows;
                // hd 128 and small grids (fewer than 128 workgroups of 128 rows) use 2
                const int64_t wg4 = ((Nq + 127) / 128) * Hq * B;
                int waves = (D == 64 && wg4 >= 128) ? 4 : 2;
                if (w.tune.waves_override == 2 || w.tune.waves_override == 4) waves = w.tune.waves_override;
                e = vxfa::launch_prefill(a, (int)D, waves, st);
            }
        }
    }
    if (e != hipSuccess) {
        set_err(w, "kernel launch: %s", hipGetErrorString(e));
        return VXFA_HIP_ERROR;
    }
    return VXFA_OK;
}

}  // namespace

extern "C" {

int vxfa_flash_attn_ext(vxfa_ctx* c, const vxfa_tensor* q, const vxfa_tensor* k, const vxfa_tensor* v,
                        const vxfa_tensor* mask, vxfa_tensor* dst, float scale, float max_bias, float logit_softcap,
                        void* stream) {
    if (!c) return VXFA_INVALID_ARG;
    Workspace w = c->view();
    return run(w, q, k, v, mask, nullptr, dst, scale, max_bias, logit_softcap, stream);
}

int vxfa_kv_append(vxfa_ctx* c, const vxfa_tensor* k_new, const vxfa_tensor* v_new, vxfa_tensor* k, vxfa_tensor* v,
                   void* stream) {
    if (!c) return VXFA_INVALID_ARG;
    c->last_error[0] = 0;
    Workspace w = c->view();
    if (!k || !v) { set_err(w, "k and v are required"); return VXFA_INVALID_ARG; }
    const char* why = nullptr;
    const int rc = check_append(k, v, k_new, v_new, &why);
    if (rc != VXFA_OK) {
        set_err(w, "%s", why);
        return rc;
    }
    hipError_t e = hipSetDevice(c->device);
    if (e != hipSuccess) { set_err(w, "hipSetDevice: %s", hipGetErrorString(e)); return VXFA_HIP_ERROR; }
    e = vxfa::launch_kv_append(append_args(k, v, k_new, v_new), reinterpret_cast<hipStream_t>(stream));
    if (e != hipSuccess) { set_err(w, "kv append: %s", hipGetErrorString(e)); return VXFA_HIP_ERROR; }
    return VXFA_OK;
}

int vxfa_flash_attn_ext_append(vxfa_ctx* c, const vxfa_tensor* q, vxfa_tensor* k, vxfa_tensor* v,
                               const vxfa_tensor* k_new, const vxfa_tensor* v_new, const vxfa_tensor* mask,
                               vxfa_tensor* dst, float scale, float max_bias, float logit_softcap, void* stream) {
    if (!c) return VXFA_INVALID_ARG;
    Workspace w = c->view();
    if (!k_new || !v_new) {
        set_err(w, "k_new and v_new are required");
        return VXFA_INVALID_ARG;
    }
    return run(w, q, k, v, mask, nullptr, dst, scale, max_bias, logit_softcap, stream, k_new, v_new);
}

int vxfa_flash_attn_ext_ring(vxfa_ctx* c, const vxfa_tensor* q, vxfa_tensor* k, vxfa_tensor* v, const vxfa_ring* ring,
                             const vxfa_tensor* k_new, const vxfa_tensor* v_new, vxfa_tensor* dst, float scale,
                             float max_bias, float logit_softcap, void* stream) {
    if (!c) return VXFA_INVALID_ARG;
    Workspace w = c->view();
    if (!ring || (k_new == nullptr) != (v_new == nullptr)) {
        set_err(w, "a ring descriptor is required; k_new and v_new come together");
        return VXFA_INVALID_ARG;
    }
    return run(w, q, k, v, nullptr, nullptr, dst, scale, max_bias, logit_softcap, stream, k_new, v_new, ring);
}

int vxfa_flash_attn_ext_rope(vxfa_ctx* c, const vxfa_tensor* q, vxfa_tensor* k, vxfa_tensor* v,
                             const vxfa_tensor* k_new, const vxfa_tensor* v_new, const vxfa_rope* rope,
                             const vxfa_tensor* mask, vxfa_tensor* dst, float scale, float max_bias,
                             float logit_softcap, void* stream) {
    if (!c) return VXFA_INVALID_ARG;
    Workspace w = c->view();
    if (!rope || !k_new || !v_new) {
        set_err(w, "rope, k_new and v_new are required");
        return VXFA_INVALID_ARG;
    }
    return run(w, q, k, v, mask, nullptr, dst, scale, max_bias, logit_softcap, stream, k_new, v_new, nullptr, rope);
}

int vxfa_check_mask_desc(const vxfa_mask_desc* m) {
    if (!m) return VXFA_OK;
    if (m->kind != VXFA_MASK_NONE && m->kind != VXFA_MASK_CAUSAL) return VXFA_INVALID_ARG;
    if (m->window < 0) return VXFA_INVALID_ARG;
    return VXFA_OK;
}

int vxfa_flash_attn_ext_implicit(vxfa_ctx* c, const vxfa_tensor* q, const vxfa_tensor* k, const vxfa_tensor* v,
                                 const vxfa_mask_desc* mask, vxfa_tensor* dst, float scale, float max_bias,
                                 float logit_softcap, void* stream) {
    if (!c) return VXFA_INVALID_ARG;
    Workspace w = c->view();
    if (vxfa_check_mask_desc(mask) != VXFA_OK) {
        set_err(w, "mask descriptor: kind must be VXFA_MASK_NONE or VXFA_MASK_CAUSAL and window >= 0");
        return VXFA_INVALID_ARG;
    }
    return run(w, q, k, v, nullptr, mask, dst, scale, max_bias, logit_softcap, stream);
}

}  // extern "C"

extern "C" {

int vxfa_flash_attn_ext_noalloc(const vxfa_tensor* q, const vxfa_tensor* k, const vxfa_tensor* v,
                                const vxfa_tensor* mask, vxfa_tensor* dst, float scale, float max_bias,
                                float logit_softcap, void* stream) {
    t_noalloc_err[0] = 0;
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess || device < 0 || device >= kMaxDevices) {
        snprintf(t_noalloc_err, sizeof(t_noalloc_err), "no usable current HIP device");
        return VXFA_HIP_ERROR;
    }
    void* ptr = nullptr;
    {
        // first call on this device (the device is current): the array's
        // device address, once. hipGetSymbolAddress may load the code object,
        // which a stream capture does not allow, so that call must be made
        // outside capture (later calls may be captured).
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        if (!g_scratch_ptr[device]) {
            hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
            if (hipStreamIsCapturing(reinterpret_cast<hipStream_t>(stream), &cs) == hipSuccess &&
                cs != hipStreamCaptureStatusNone) {
                snprintf(t_noalloc_err, sizeof(t_noalloc_err),
                         "the first no-alloc call on a device must be made outside stream capture");
                return VXFA_HIP_ERROR;
            }
            e = hipGetSymbolAddress(&g_scratch_ptr[device], HIP_SYMBOL(scratch));
            if (e != hipSuccess || !g_scratch_ptr[device]) {
                g_scratch_ptr[device] = nullptr;
                snprintf(t_noalloc_err, sizeof(t_noalloc_err), "hipGetSymbolAddress(scratch): %s",
                         hipGetErrorString(e));
                return VXFA_HIP_ERROR;
            }
        }
        ptr = g_scratch_ptr[device];
    }
    // the tuning variables, read once per process
    static const Tuning tune = [] {
        Tuning t;
        t.read_env();
        return t;
    }();
    // records (decode) and staging (prefill with F32 K/V) are never needed
    // by one call together: both use the whole array
    Workspace w{device, static_cast<float*>(ptr), kScratchBytes, static_cast<_Float16*>(ptr), kScratchBytes,
                t_noalloc_err, sizeof(t_noalloc_err), tune};
    return run(w, q, k, v, mask, nullptr, dst, scale, max_bias, logit_softcap, stream);
}

}  // extern "C"
