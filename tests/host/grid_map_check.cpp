// Host check of the kernels' index helpers in fa_common.h (built by
// tests/test_grid_map.py, no GPU): FastDiv against the / operator, and
// GridMap::locate against the plain XCD-aware decomposition
//   gidx = xcd < r8 ? xcd (q8 + 1) : r8 (q8 + 1) + (xcd - r8) q8, + lin / 8
//   qt = gidx % nqt, h = gidx / nqt % hq, b = gidx / (nqt hq),
//   hk = h / (hq / hkv), bkv = b / (B / bk)
// and that the map is a bijection of [0, nwg) onto the (qt, h, b) triples;
// and the F32 K/V staging kernel's split of its flat index i (8-element
// groups of a [b][n][h][d] buffer) into (row, element, kv head, position,
// batch) by shifts and DivMod, against the plain division.
#include "../../voxtral.cpp_amd/csrc/fa_common.h"
#include <cstdio>
#include <cstdlib>
#include <vector>

using vxfa::FastDiv;
using vxfa::GridMap;

static int fail(const char* what, uint64_t a, uint64_t b, uint64_t c) {
    printf("FAIL %s: %llu %llu %llu\n", what, (unsigned long long)a, (unsigned long long)b, (unsigned long long)c);
    return 1;
}

int main() {
    uint64_t rng = 0x9e3779b97f4a7c15ull;
    auto next = [&]() { rng ^= rng << 13; rng ^= rng >> 7; rng ^= rng << 17; return rng; };
    // divisors: 1 .. 5000, powers of two and their neighbours, large values
    std::vector<uint32_t> ds;
    for (uint32_t d = 1; d <= 5000; ++d) ds.push_back(d);
    for (int k = 1; k < 31; ++k) for (int e = -1; e <= 1; ++e) ds.push_back((1u << k) + e);
    for (int i = 0; i < 2000; ++i) ds.push_back(1 + (uint32_t)(next() % 0x7fffffffu));
    long checks = 0;
    for (uint32_t d : ds) {
        if (d == 0) continue;
        const FastDiv f = FastDiv::make(d);
        std::vector<uint32_t> ns = {0, 1, 2, d - 1, d, d + 1, 0x7fffffffu, 0x7ffffffeu};
        for (int i = 0; i < 64; ++i) ns.push_back((uint32_t)(next() % 0x80000000ull));
        for (uint32_t q : {1u, 2u, 3u, 1000u, 0x7fffffffu / d}) {   // multiples of d and their neighbours
            const uint64_t m = (uint64_t)q * d;
            for (int e = -1; e <= 1; ++e)
                if ((int64_t)m + e >= 0 && (int64_t)m + e < 0x80000000ll) ns.push_back((uint32_t)(m + e));
        }
        for (uint32_t n : ns) {
            if (n >= 0x80000000u) continue;
            if (f.div(n) != n / d) return fail("FastDiv", n, d, f.div(n));
            ++checks;
        }
        if (d <= 3000)
            for (uint32_t n = 0; n < 3 * d + 64; ++n) {
                if (f.div(n) != n / d) return fail("FastDiv dense", n, d, f.div(n));
                ++checks;
            }
    }
    // grids: query tiles x heads x batches, with GQA and kv-batch broadcast
    const int shapes[][5] = {{12, 20, 1, 20, 1}, {1, 1, 1, 1, 1}, {3, 32, 1, 8, 1}, {7, 32, 2, 8, 2},
                             {5, 8, 4, 2, 1}, {1, 32, 32, 8, 32}, {13, 3, 5, 3, 5}, {2, 4, 6, 1, 3},
                             {24, 20, 1, 20, 1}, {1, 1, 9, 1, 1}, {8, 16, 3, 4, 3}};
    for (auto& s : shapes) {
        const int nqt = s[0], hq = s[1], B = s[2], hkv = s[3], bk = s[4];
        const int nwg = nqt * hq * B;
        const GridMap g = GridMap::make(nwg, nqt, hq, hkv, B, bk);
        const int q8 = nwg >> 3, r8 = nwg & 7;
        std::vector<int> seen((size_t)nwg, 0);
        for (int lin = 0; lin < nwg; ++lin) {
            const int xcd = lin & 7;
            const int gidx = (xcd < r8 ? xcd * (q8 + 1) : r8 * (q8 + 1) + (xcd - r8) * q8) + (lin >> 3);
            int qt, h, b, hk, bkv;
            g.locate((uint32_t)lin, qt, h, b, hk, bkv);
            if (qt != gidx % nqt || h != (gidx / nqt) % hq || b != gidx / (nqt * hq)) return fail("locate", lin, gidx, nwg);
            if (hk != h / (hq / hkv) || bkv != b / (B / bk)) return fail("locate kv", lin, hk, bkv);
            if (gidx < 0 || gidx >= nwg || seen[gidx]++) return fail("bijection", lin, gidx, nwg);
            ++checks;
        }
    }
    // the heavy-first order (make_tiles_desc) where hq * B is a multiple of 8:
    // XCD x = lin % 8 takes pairs t in [x hx, (x + 1) hx), tile nqt - 1 - j / hx
    // for j = lin / 8, t = x hx + j % hx; a bijection onto the (qt, h, b) triples
    const int dshapes[][5] = {{12, 32, 1, 32, 1}, {12, 20, 2, 20, 2}, {1, 8, 1, 8, 1}, {5, 16, 3, 4, 3},
                              {24, 32, 1, 8, 1}, {3, 4, 2, 2, 1}, {12, 20, 1, 20, 1}};
    for (auto& s : dshapes) {
        const int nqt = s[0], hq = s[1], B = s[2], hkv = s[3], bk = s[4];
        const int nwg = nqt * hq * B;
        const GridMap g = GridMap::make_tiles_desc(nwg, nqt, hq, hkv, B, bk);
        const bool desc = (hq * B) % 8 == 0;
        if ((g.hx != 0) != desc) return fail("desc eligibility", hq, B, g.hx);
        const int hx = hq * B / 8;
        std::vector<int> seen((size_t)nwg, 0);
        for (int lin = 0; lin < nwg; ++lin) {
            int qt, h, b, hk, bkv;
            g.locate((uint32_t)lin, qt, h, b, hk, bkv);
            int wqt, wt;
            if (desc) {
                const int x = lin & 7, j = lin >> 3;
                wqt = nqt - 1 - j / hx;
                wt = x * hx + j % hx;
            } else {
                const int q8 = nwg >> 3, r8 = nwg & 7, xcd = lin & 7;
                const int gidx = (xcd < r8 ? xcd * (q8 + 1) : r8 * (q8 + 1) + (xcd - r8) * q8) + (lin >> 3);
                wqt = gidx % nqt;
                wt = gidx / nqt;
            }
            if (qt != wqt || h != wt % hq || b != wt / hq) return fail("locate desc", lin, qt, wqt);
            if (hk != h / (hq / hkv) || bkv != b / (B / bk)) return fail("locate desc kv", lin, hk, bkv);
            const int gi = (b * hq + h) * nqt + qt;
            if (qt < 0 || qt >= nqt || gi < 0 || gi >= nwg || seen[gi]++) return fail("bijection desc", lin, gi, nwg);
            ++checks;
        }
    }
    // staging index (to_f16_kv_kernel): i -> r = i >> log2(d/8), e = 8 (i - r (d/8)),
    // hh = r % h, pos = (r / h) % n, bb = r / h / n; element 8 i of the buffer
    const int stg[][4] = {{64, 1500, 20, 1}, {128, 439, 8, 1}, {64, 7, 3, 5}, {128, 8192, 8, 2}, {64, 1, 1, 1}};
    for (auto& s4 : stg) {
        const uint32_t d = s4[0], n = s4[1], h = s4[2], b = s4[3];
        uint32_t l2 = 0;
        while ((1u << l2) < d / 8) ++l2;
        const vxfa::DivMod dh = vxfa::DivMod::make(h), dn = vxfa::DivMod::make(n);
        const uint32_t total8 = b * n * h * (d / 8);
        for (uint32_t i = 0; i < total8; ++i) {
            const uint32_t r = i >> l2, e = (i - (r << l2)) * 8;
            const uint32_t r2 = dh.div(r), hh = r - r2 * dh.d, bb = dn.div(r2), pos = r2 - bb * dn.d;
            if (bb >= b || pos >= n || hh >= h || e >= d) return fail("stage range", i, d, n);
            if ((uint64_t)i * 8 != (((uint64_t)bb * n + pos) * h + hh) * d + e) return fail("stage index", i, d, n);
            ++checks;
        }
    }
    printf("ok %ld\n", checks);
    return 0;
}
