// Host-side fuzz of the C ABI's contract validation (vxfa_supports, the
// supports_op analogue) under AddressSanitizer and UndefinedBehaviorSanitizer:
// random descriptors (shapes, strides, types, null pointers, odd alignments,
// huge extents) must come back as a status code, never crash or trip a
// sanitizer. Built by tests/test_sanitizers.py; host code only (no kernel is
// launched and no GPU is needed).
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>

#include "../../include/vxfa.h"
#include "../../voxtral.cpp_amd/csrc/fa_common.h"

// The kernels' host launchers, stubbed: validation never reaches a launch,
// and leaving the device code out keeps this build to the host shim.
namespace vxfa {
hipError_t launch_decode(const AttnArgs&, int, int, hipStream_t) { return hipErrorInvalidValue; }
hipError_t launch_prefill(const AttnArgs&, int, int, hipStream_t) { return hipErrorInvalidValue; }
hipError_t launch_prefill64_pp(const AttnArgs&, const StageReq*, hipStream_t) { return hipErrorInvalidValue; }
hipError_t launch_prefill_pair(const AttnArgs&, hipStream_t) { return hipErrorInvalidValue; }
hipError_t launch_mask_prep(const AttnArgs&, const StageReq*, hipStream_t) { return hipErrorInvalidValue; }
bool prefill_pair_fits(const AttnArgs&) { return true; }
hipError_t launch_zero(float*, int64_t, hipStream_t) { return hipErrorInvalidValue; }
hipError_t launch_kv_append(const AppendArgs&, hipStream_t) { return hipErrorInvalidValue; }
hipError_t launch_to_f16_kv(const StageReq&, hipStream_t) { return hipErrorInvalidValue; }
}  // namespace vxfa

static int64_t pick(std::mt19937_64& g, const int64_t* v, int n) { return v[g() % n]; }

int main(int argc, char** argv) {
    const int iters = argc > 1 ? atoi(argv[1]) : 200000;
    std::mt19937_64 g(12345);
    static const int64_t dims[] = {0, 1, 2, 7, 8, 31, 32, 64, 128, 256, 439, 1500, 8192, 65535, 65536,
                                   (int64_t)1 << 31, -1, INT64_MAX};
    static const int32_t types[] = {VXFA_TYPE_F32, VXFA_TYPE_F16, 2, -1, 39};
    alignas(64) static unsigned char buf[4096];
    int counts[8] = {0};
    for (int it = 0; it < iters; ++it) {
        vxfa_tensor t[5];
        for (int i = 0; i < 5; ++i) {
            std::memset(&t[i], 0, sizeof(t[i]));
            t[i].type = types[g() % 5];
            t[i].data = (g() % 8) ? (void*)(buf + (g() % 3 == 0 ? (g() % 64) : 0)) : nullptr;
            for (int d = 0; d < 4; ++d) {
                t[i].ne[d] = (g() % 3) ? pick(g, dims, 11) : pick(g, dims, 18);
                t[i].nb[d] = (size_t)((g() % 4) ? pick(g, dims, 13) * (d == 0 ? 1 : 2) : (int64_t)(g() % 100000));
            }
            if (g() % 2) {   // a consistent contiguous layout half of the time
                const int64_t el = t[i].type == VXFA_TYPE_F32 ? 4 : 2;
                t[i].nb[0] = el;
                for (int d = 1; d < 4; ++d) t[i].nb[d] = t[i].nb[d - 1] * (size_t)(t[i].ne[d - 1] > 0 ? t[i].ne[d - 1] : 1);
            }
        }
        const float scales[] = {0.125f, 0.f, -1.f, 1e30f, __builtin_inff(), __builtin_nanf("")};
        const int rc = vxfa_supports(&t[0], &t[1], &t[2], (g() % 3) ? nullptr : &t[3], (g() % 10) ? &t[4] : nullptr,
                                     scales[g() % 6], (g() % 5) ? 0.f : 1.f, (g() % 5) ? 0.f : 30.f);
        if (rc < 0 || rc > 7) { std::printf("bad status %d\n", rc); return 1; }
        counts[rc]++;
        (void)vxfa_status_str(rc);
        vxfa_mask_desc md{(int32_t)(g() % 4) - 1, (int32_t)(g() % 5) - 2, (int64_t)(g() % 7) - 3};
        (void)vxfa_check_mask_desc(&md);
    }
    (void)vxfa_check_mask_desc(nullptr);
    (void)vxfa_last_error(nullptr);
    std::printf("ok %d %d %d %d\n", counts[0], counts[1], counts[2], counts[3]);
    return 0;
}
