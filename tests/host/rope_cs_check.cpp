// Host check of the rotary embedding's cos / sin (rope_cs of fa_common.h,
// built by tests/test_rope_cs.py, no GPU): for the angles ggml's running
// product gives (theta_0 = p, theta_{j+1} = theta_j * ts in float, ts =
// powf(base, -2 / n_dims)) at positions up to 2^20 and for plain angles
// over [-1000, 1000], the (cos, sin) pair against libm's double-precision
// cos / sin of the same float angle. Prints the largest absolute error.
#include "../../voxtral.cpp_amd/csrc/fa_common.h"
#include <cmath>
#include <cstdio>

int main() {
    double worst = 0.0, worst_th = 0.0;
    auto check = [&](float th, float2 cs) {
        const double c = std::cos((double)th), s = std::sin((double)th);
        const double e = std::fmax(std::fabs(cs.x - c), std::fabs(cs.y - s));
        if (e > worst) { worst = e; worst_th = th; }
    };
    const int positions[] = {0, 1, 2, 3, 7, 63, 100, 439, 511, 1023, 4095, 8191, 16383, 65535, 1 << 20};
    const float bases[] = {1.0e4f, 1.0e6f, 500.0f};
    const int dims[] = {128, 64};
    for (float base : bases)
        for (int nd : dims) {
            const float ts = powf(base, -2.0f / (float)nd);
            for (int p : positions) {
                float th = (float)p;
                for (int j = 0; j < nd / 2; ++j) {
                    check(th, vxfa::rope_cs(p, j, ts));
                    th *= ts;
                }
            }
        }
    for (int i = -200000; i <= 200000; ++i) {
        const float th = (float)i * 0.005f;
        check(th, vxfa::rope_cs_of_angle(th));
    }
    printf("%s max abs error %.3e at angle %.6g\n", worst < 1e-6 ? "ok" : "FAIL", worst, worst_th);
    return worst < 1e-6 ? 0 : 1;
}
