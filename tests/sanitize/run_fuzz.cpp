// Host-side fuzz of every entry point's run path (vxfa_api.cpp: validation,
// routing, split choice, workspace placement, F32 staging, implicit masks,
// ring buffers, appends, rotary embedding, the no-alloc scratch) under
// AddressSanitizer and UndefinedBehaviorSanitizer, with no GPU: the HIP
// runtime calls the path makes (device selection, the context's one
// allocation, the scratch symbol lookup, the capture query) are replaced by
// host stand-ins, and the kernels' host launchers by stubs that check what
// the kernels assume of their arguments instead of launching:
//   * decode: 1 <= n_split <= 64, and the split records of every (batch,
//     kv head) pair inside one workspace allocation;
//   * F32 staging: both f16 copies inside one allocation, disjoint;
//   * pipelined hd 64 prefill with a mask tensor: the interval table inside
//     one allocation and clear of the staged K/V;
//   * every launch: positive sizes, non-null operands.
// Descriptors are voxtral-shaped (decode, decoder prefill, encoder, realtime
// encoder, batched streams) with random sizes, types, strides, alignments,
// masks and broadcast planes; most are valid, so the calls reach the
// launchers. Built and run by tests/test_sanitizers.py.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "../../include/vxfa.h"
#include "../../voxtral.cpp_amd/csrc/fa_common.h"

// ---- host stand-ins for the HIP runtime --------------------------------------
namespace {
struct Alloc {
    uintptr_t lo, hi;
};
std::vector<Alloc> g_allocs;
alignas(256) unsigned char g_scratch_stand_in[(size_t)8 << 20];
int g_fail = 0;
size_t g_launches = 0;

void fail(const char* what) {
    std::printf("violation: %s\n", what);
    g_fail = 1;
}
bool inside_one(const void* p, size_t bytes) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    for (const Alloc& r : g_allocs)
        if (a >= r.lo && a + bytes <= r.hi) return true;
    return false;
}
// byte ranges written by the last F32 staging launch (cleared per call)
uintptr_t g_stage_lo = 0, g_stage_hi = 0;
}  // namespace

extern "C" {
hipError_t hipGetDeviceCount(int* n) {
    *n = 1;
    return hipSuccess;
}
hipError_t hipGetDevice(int* d) {
    *d = 0;
    return hipSuccess;
}
hipError_t hipSetDevice(int d) { return d == 0 ? hipSuccess : hipErrorInvalidDevice; }
hipError_t hipMalloc(void** p, size_t n) {
    *p = std::malloc(n);
    if (!*p) return hipErrorOutOfMemory;
    g_allocs.push_back({reinterpret_cast<uintptr_t>(*p), reinterpret_cast<uintptr_t>(*p) + n});
    return hipSuccess;
}
hipError_t hipFree(void* p) {
    for (size_t i = 0; i < g_allocs.size(); ++i)
        if (g_allocs[i].lo == reinterpret_cast<uintptr_t>(p)) g_allocs.erase(g_allocs.begin() + (long)i);
    std::free(p);
    return hipSuccess;
}
hipError_t hipDeviceSynchronize(void) { return hipSuccess; }
hipError_t hipStreamIsCapturing(hipStream_t, hipStreamCaptureStatus* s) {
    *s = hipStreamCaptureStatusNone;
    return hipSuccess;
}
hipError_t hipGetSymbolAddress(void** p, const void*) {
    *p = g_scratch_stand_in;
    const uintptr_t lo = reinterpret_cast<uintptr_t>(g_scratch_stand_in);
    bool known = false;
    for (const Alloc& r : g_allocs) known = known || r.lo == lo;
    if (!known) g_allocs.push_back({lo, lo + sizeof(g_scratch_stand_in)});
    return hipSuccess;
}
}

// ---- the kernels' host launchers, as argument checks -------------------------
namespace vxfa {
static void common(const AttnArgs& a) {
    ++g_launches;
    if (a.nq <= 0 || a.nkv <= 0 || a.hq <= 0 || a.hkv <= 0 || a.b <= 0 || a.bk <= 0) fail("non-positive size");
    if (!a.q || !a.k || !a.v || !a.dst) fail("null operand");
    if (a.hq % a.hkv || a.b % a.bk) fail("broadcast");
}
static void check_stage(const StageReq& r) {
    const size_t bytes = (size_t)r.d * r.n * r.h * r.b * 2;
    if (!r.k || !r.v) fail("staging source");
    if (!inside_one(r.dk, bytes) || !inside_one(r.dv, bytes)) fail("staging outside the workspace");
    const uintptr_t a = reinterpret_cast<uintptr_t>(r.dk), c = reinterpret_cast<uintptr_t>(r.dv);
    if (a < c + bytes && c < a + bytes) fail("staged K and V overlap");
    g_stage_lo = a < c ? a : c;
    g_stage_hi = (a < c ? c : a) + bytes;
}
hipError_t launch_to_f16_kv(const StageReq& r, hipStream_t) {
    ++g_launches;
    check_stage(r);
    return hipSuccess;
}
hipError_t launch_decode(const AttnArgs& a, int D, int G, hipStream_t) {
    common(a);
    if (a.n_split < 1 || a.n_split > kDecodeMaxSplit) fail("n_split out of range");
    if (G != a.hq / a.hkv) fail("group");
    if (a.n_split > 1) {
        const size_t bytes = (size_t)a.b * a.hkv * a.n_split * dec_record_floats(D, G) * sizeof(float);
        if (!a.ws || !inside_one(a.ws, bytes)) fail("decode records outside the workspace");
    }
    return hipSuccess;
}
hipError_t launch_prefill(const AttnArgs& a, int, int, hipStream_t) {
    common(a);
    return hipSuccess;
}
void check_mask_table(const AttnArgs& a) {
    const size_t bytes = (size_t)a.nq * a.hm * a.bm * 8;
    if (!a.mask_rows || !inside_one(a.mask_rows, bytes)) fail("mask interval table outside the workspace");
    const uintptr_t lo = reinterpret_cast<uintptr_t>(a.mask_rows);
    if (g_stage_hi > g_stage_lo && lo < g_stage_hi && g_stage_lo < lo + bytes)
        fail("mask interval table overlaps the staged K/V");
}
hipError_t launch_mask_prep(const AttnArgs& a, const StageReq* stage, hipStream_t) {
    ++g_launches;
    if (stage) check_stage(*stage);
    if (!a.mask) fail("mask pre-pass without a mask");
    check_mask_table(a);
    return hipSuccess;
}
hipError_t launch_prefill64_pp(const AttnArgs& a, const StageReq* stage, hipStream_t) {
    if (stage) check_stage(*stage);
    common(a);
    if (a.mask) check_mask_table(a);
    return hipSuccess;
}
hipError_t launch_prefill_pair(const AttnArgs& a, hipStream_t) {
    common(a);
    if (a.mask_rows) {
        // the interval table is only read after the pre-pass that fills it
        if (!a.mask) fail("interval table without a mask");
        check_mask_table(a);
    }
    return hipSuccess;
}
bool prefill_pair_fits(const AttnArgs&) { return true; }
hipError_t launch_zero(float* p, int64_t n, hipStream_t) {
    ++g_launches;
    if (!p || n <= 0) fail("zero fill");
    return hipSuccess;
}
hipError_t launch_kv_append(const AppendArgs&, hipStream_t) {
    ++g_launches;
    return hipSuccess;
}
}  // namespace vxfa

// ---- voxtral-shaped random descriptors -----------------------------------------
namespace {
uintptr_t fake_addr(std::mt19937_64& g, int align) {
    // never dereferenced on the host: device addresses in a high range
    return ((uintptr_t)0x7e0000000000ull + (g() % 4096) * 4096) + (uintptr_t)align;
}
vxfa_tensor tensor(uintptr_t data, int type, int64_t n0, int64_t n1, int64_t n2, int64_t n3, size_t nb1, size_t nb2,
                   size_t nb3) {
    vxfa_tensor t;
    std::memset(&t, 0, sizeof(t));
    t.data = reinterpret_cast<void*>(data);
    t.type = type;
    t.ne[0] = n0; t.ne[1] = n1; t.ne[2] = n2; t.ne[3] = n3;
    t.nb[0] = type == VXFA_TYPE_F32 ? 4 : 2;
    t.nb[1] = nb1; t.nb[2] = nb2; t.nb[3] = nb3;
    return t;
}
template <class T>
T pick(std::mt19937_64& g, std::initializer_list<T> v) {
    return v.begin()[g() % v.size()];
}
}  // namespace

int main(int argc, char** argv) {
    const int iters = argc > 1 ? atoi(argv[1]) : 20000;
    std::setvbuf(stdout, nullptr, _IONBF, 0);
    std::mt19937_64 g(777);
    vxfa_ctx* ctx = vxfa_ctx_create(0);
    if (!ctx) { std::printf("no context\n"); return 1; }
    int counts[8] = {0};
    for (int it = 0; it < iters; ++it) {
        g_stage_lo = g_stage_hi = 0;
        const int64_t D = pick<int64_t>(g, {64, 128, 128, 80});
        const int64_t Hkv = pick<int64_t>(g, {1, 2, 8, 20, 32});
        const int64_t G = pick<int64_t>(g, {1, 2, 4, 3});
        const int64_t Hq = Hkv * G;
        const int64_t B = pick<int64_t>(g, {1, 1, 2, 3});
        const int64_t Bk = (g() % 2) ? 1 : B;
        const int64_t Nq = pick<int64_t>(g, {0, 1, 1, 2, 31, 64, 130, 439, 1500});
        const int64_t Nkv = pick<int64_t>(g, {0, 1, 33, 300, 439, 1500, 8192, 16384});
        const int64_t cap = Nkv + (int64_t)(g() % 3) * 64;
        const int kvt = (g() % 3) ? VXFA_TYPE_F16 : VXFA_TYPE_F32;
        const int qt = (g() % 4) ? VXFA_TYPE_F32 : VXFA_TYPE_F16;
        const size_t ke = kvt == VXFA_TYPE_F32 ? 4 : 2, qe = qt == VXFA_TYPE_F32 ? 4 : 2;
        // q [D, Nq, Hq, B]: token-major rows (decoder) or head-major (encoder)
        vxfa_tensor q = tensor(fake_addr(g, 0), qt, D, Nq, Hq, B, Hq * D * qe, D * qe, Nq * Hq * D * qe);
        vxfa_tensor k = tensor(fake_addr(g, 0), kvt, D, Nkv, Hkv, Bk, Hkv * D * ke, D * ke, cap * Hkv * D * ke);
        vxfa_tensor v = tensor(fake_addr(g, 0), kvt, D, Nkv, Hkv, Bk, Hkv * D * ke, D * ke, cap * Hkv * D * ke);
        vxfa_tensor dst = tensor(fake_addr(g, 0), VXFA_TYPE_F32, D, Hq, Nq, B, D * 4, Hq * D * 4, Nq * Hq * D * 4);
        // mask: none, [Nkv, Nq(+pad), Hm, Bm], any 2-byte alignment
        const int mk = (int)(g() % 3);
        const int64_t Hm = (g() % 3) ? 1 : Hq, Bm = (g() % 2) ? 1 : B;
        const int64_t mrows = Nq + (int64_t)(g() % 2) * 7;
        const size_t mrow_b = (size_t)Nkv * 2 + (g() % 2) * 16;
        vxfa_tensor m = tensor(fake_addr(g, (int)(g() % 8) * 2), VXFA_TYPE_F16, Nkv, mrows, Hm, Bm, mrow_b,
                               mrow_b * mrows, mrow_b * mrows * Hm);
        const float scale = pick<float>(g, {0.125f, 0.0883883f, 0.f, -0.125f});
        void* stream = nullptr;
        int rc = 0;
        switch (g() % 7) {
            case 0:
            case 1:
                rc = vxfa_flash_attn_ext(ctx, &q, &k, &v, mk ? &m : nullptr, &dst, scale, 0.f, 0.f, stream);
                break;
            case 2: {
                vxfa_mask_desc md{VXFA_MASK_CAUSAL, pick<int32_t>(g, {0, 1, 31, 750}),
                                  pick<int64_t>(g, {0, Nkv - Nq, Nkv - 1, -5, Nkv + 3})};
                rc = vxfa_flash_attn_ext_implicit(ctx, &q, &k, &v, &md, &dst, scale, 0.f, 0.f, stream);
                break;
            }
            case 3: {
                const int64_t nn = pick<int64_t>(g, {1, 1, 2, Nq});
                vxfa_tensor kn = tensor(fake_addr(g, 0), VXFA_TYPE_F32, Hkv * D, nn, 1, Bk, Hkv * D * 4,
                                        nn * Hkv * D * 4, nn * Hkv * D * 4);
                vxfa_tensor vn = kn;
                vn.data = reinterpret_cast<void*>(fake_addr(g, 0));
                k.type = v.type = VXFA_TYPE_F16;
                rc = vxfa_flash_attn_ext_append(ctx, &q, &k, &v, &kn, &vn, mk ? &m : nullptr, &dst, scale, 0.f, 0.f,
                                                stream);
                break;
            }
            case 4: {
                vxfa_ring r{(int64_t)(g() % (cap + 1)), (int64_t)(g() % (cap + 1))};
                vxfa_tensor kn = tensor(fake_addr(g, 0), VXFA_TYPE_F32, Hkv * D, 1, 1, Bk, Hkv * D * 4, Hkv * D * 4,
                                        Hkv * D * 4);
                k.ne[1] = v.ne[1] = cap;
                k.type = v.type = VXFA_TYPE_F16;
                rc = vxfa_flash_attn_ext_ring(ctx, &q, &k, &v, &r, (g() % 2) ? &kn : nullptr, (g() % 2) ? &kn : nullptr,
                                              &dst, scale, 0.f, 0.f, stream);
                break;
            }
            case 5: {
                vxfa_tensor kn = tensor(fake_addr(g, 0), VXFA_TYPE_F32, Hkv * D, Nq, 1, Bk, Hkv * D * 4,
                                        Nq * Hkv * D * 4, Nq * Hkv * D * 4);
                vxfa_rope rp{reinterpret_cast<const int32_t*>(fake_addr(g, 0)), (int32_t)pick<int64_t>(g, {D, 64, 0}),
                             0, 1e6f, 1.0f};
                k.type = v.type = VXFA_TYPE_F16;
                rc = vxfa_flash_attn_ext_rope(ctx, &q, &k, &v, &kn, &kn, &rp, mk ? &m : nullptr, &dst, scale, 0.f,
                                              0.f, stream);
                break;
            }
            default:
                rc = vxfa_flash_attn_ext_noalloc(&q, &k, &v, mk ? &m : nullptr, &dst, scale, 0.f, 0.f, stream);
                break;
        }
        if (rc < 0 || rc > 7) {
            std::printf("bad status %d\n", rc);
            g_fail = 1;
        } else {
            counts[rc]++;
        }
        (void)vxfa_last_error(ctx);
        if (g_fail) {
            std::printf("iteration %d: D %lld Hq %lld Hkv %lld B %lld Bk %lld Nq %lld Nkv %lld kv %d mask %d\n", it,
                        (long long)D, (long long)Hq, (long long)Hkv, (long long)B, (long long)Bk, (long long)Nq,
                        (long long)Nkv, kvt, mk);
            break;
        }
    }
    vxfa_ctx_destroy(ctx);
    std::printf("ok %d %d %d %d %d launches %zu\n", counts[0], counts[1], counts[2], counts[3], counts[4], g_launches);
    return g_fail;
}
