// Host-side check of the prefill contraction's work plan (G16Plan): compiled by tests/test_g16_plan.py, no GPU.
#include "vq_gemm16_impl.h"
#include <cstdio>
#include <vector>
using namespace vq;
int main() {
    long bad = 0, cases = 0, hybrid = 0;
    for (int cus : {256, 304, 80, 8})
    for (int rows : {64, 256, 1000, 5120, 10240, 17408, 248320 / 8})
    for (int cols : {256, 512, 5120, 17408})
    for (int M : {1, 37, 128, 300, 512, 1024, 4096})
    for (int inv = 0; inv < 2; ++inv) {
        const G16Plan p = g16_plan(rows, cols, M, cus, inv);
        ++cases; if (p.D) ++hybrid;
        std::vector<int> cover(p.U, 0), owner(p.U, -1);
        std::vector<std::vector<int>> segs(p.tiles);  // workgroups with a part of tile t
        for (int v = 0; v < p.W; ++v) {
            long ue = p.dp1(v), u = p.dp0(v);
            bool whole = u < ue;
            if (!whole) u = p.u0(v), ue = p.u0(v + 1);
            while (u < ue) {
                const int tile = u / p.nsb, sb0 = u - (long)tile * p.nsb;
                const int sb1 = ue - u < p.nsb - sb0 ? sb0 + (int)(ue - u) : p.nsb;
                for (long x = u; x < u + (sb1 - sb0); ++x) { cover[x]++; owner[x] = v; }
                if (!(sb0 == 0 && sb1 == p.nsb)) {
                    const int k = v - p.wg_of((long)tile * p.nsb);
                    if (tile < p.t0 || k < 0 || k >= p.maxseg) { ++bad; printf("slot %d %d %d %d: tile %d t0 %d k %d maxseg %d\n", cus, rows, cols, M, tile, p.t0, k, p.maxseg); }
                    segs[tile].push_back(k);
                }
                u += sb1 - sb0;
                if (whole && u >= ue) whole = false, u = p.u0(v), ue = p.u0(v + 1);
            }
        }
        for (long x = 0; x < p.U; ++x) {
            if (cover[x] != 1) { ++bad; if (bad < 20) printf("cover %d %d %d %d inv %d: unit %ld x%d\n", cus, rows, cols, M, inv, x, cover[x]); break; }
            if (p.wg_of(x) != owner[x]) { ++bad; if (bad < 20) printf("owner %d %d %d %d inv %d: unit %ld wg_of %d owner %d\n", cus, rows, cols, M, inv, x, p.wg_of(x), owner[x]); break; }
        }
        for (int t = 0; t < p.tiles; ++t) {
            const int k0 = p.wg_of((long)t * p.nsb), k1 = p.wg_of((long)t * p.nsb + p.nsb - 1);
            const int n = k1 == k0 ? 0 : k1 - k0 + 1;
            if ((int)segs[t].size() != n) { ++bad; if (bad < 20) printf("segs %d %d %d %d: tile %d has %zu parts, reduce expects %d\n", cus, rows, cols, M, t, segs[t].size(), n); }
            for (size_t i = 0; i < segs[t].size(); ++i) if (segs[t][i] != (int)i) { ++bad; break; }
        }
        const G16Ws l = g16_layout(cols, M, p);
        if (l.total - l.part < (size_t)(p.tiles - p.t0) * p.maxseg * kG16TileFloats * 4) ++bad;
    }
    printf("cases %ld hybrid %ld bad %ld\n", cases, hybrid, bad);
    const G16Plan q = g16_plan(17408, 5120, 512, 256, false);
    printf("17408x5120 M512: tiles %d W %d rounds %d t0 %d D %ld U %ld maxseg %d slots %d\n", q.tiles, q.W, q.rounds, q.t0, q.D, q.U, q.maxseg, (q.tiles - q.t0) * q.maxseg);
    return bad != 0;
}
