// Host-side checks of the K/V tile image layout (codon-infer_amd/csrc/kv_image.h),
// run by tests/test_kv_layout.py: every element has its own bytes inside the
// image, a head group's K dims (both limbs) and a V dim's 32 keys (both limbs)
// each fill one aligned line, and the chunks attention's MFMA operand reads
// take from LDS are free of bank conflicts on a 64-bank (16 lanes per
// ds_read_b128) and a 32-bank (8 lanes) LDS.
#include <cstdio>
#include <set>
#include <vector>

#include "../../codon-infer_amd/csrc/kv_image.h"

using namespace cih;

static int fails = 0;
#define CHECK(c, ...)                         \
    do {                                      \
        if (!(c)) {                           \
            std::printf("FAIL " __VA_ARGS__); \
            std::printf("\n");                \
            fails++;                          \
        }                                     \
    } while (0)

// max lanes of one group hitting the same bank
static int conflicts(const std::vector<int> &addr, int banks, int group) {
    int worst = 1;
    for (size_t g0 = 0; g0 + group <= addr.size(); g0 += group) {
        std::vector<std::set<int>> words(banks);
        for (int l = 0; l < group; l++)
            for (int w = 0; w < 4; w++) words[(addr[g0 + l] / 4 + w) % banks].insert(addr[g0 + l] / 4 + w);
        for (auto &s : words) worst = worst > (int)s.size() ? worst : (int)s.size();
    }
    return worst;
}

template <int HD> void check() {
    using I = KvImg<HD>;
    std::vector<int> used(I::TB / 2, 0);
    for (int key = 0; key < 32; key++)
        for (int dim = 0; dim < I::HDP; dim++)
            for (int limb = 0; limb < 2; limb++) {
                const int o = I::koff(key, dim, limb);
                CHECK(o >= 0 && o < I::VOFF && o % 2 == 0, "hd %d K offset %d", HD, o);
                if (o >= 0 && o < I::TB) used[o / 2]++;
                // a group's dims of both limbs share one aligned line of 4 * GS bytes
                const int line = I::koff(key, dim / I::GS * I::GS, 0) / (4 * I::GS);
                CHECK(o / (4 * I::GS) == line, "hd %d K line key %d dim %d", HD, key, dim);
            }
    for (int key = 0; key < 32; key++)
        for (int dim = 0; dim < I::VW; dim++)
            for (int limb = 0; limb < 2; limb++) {
                const int o = I::voff(key, dim, limb);
                CHECK(o >= I::VOFF && o < I::TB && o % 2 == 0, "hd %d V offset %d", HD, o);
                if (o >= 0 && o < I::TB) used[o / 2]++;
                CHECK(o / 128 == I::voff(0, dim, 0) / 128, "hd %d V line dim %d", HD, dim);
            }
    for (size_t i = 0; i < used.size(); i++) CHECK(used[i] == 1, "hd %d byte %zu used %d times", HD, 2 * i, used[i]);
    // attention's reads: K row li, dims 16c + 8hh..; V row 32t + li, positions 16c + 8hh..
    for (int c = 0; c < I::HDP / 16; c++)
        for (int limb = 0; limb < 2; limb++) {
            std::vector<int> a(64);
            for (int lane = 0; lane < 64; lane++) {
                const int li = lane & 31, hh = lane >> 5;
                a[lane] = li * I::KRP + I::kchunk(li, I::klc(16 * c + 8 * hh, limb)) * 16;
            }
            CHECK(conflicts(a, 64, 16) == 1 && conflicts(a, 32, 8) == 1, "hd %d K read c %d limb %d conflicts", HD, c,
                  limb);
        }
    for (int t = 0; t < I::VW / 32; t++)
        for (int c = 0; c < 2; c++)
            for (int limb = 0; limb < 2; limb++) {
                std::vector<int> a(64);
                for (int lane = 0; lane < 64; lane++) {
                    const int li = lane & 31, hh = lane >> 5, row = 32 * t + li;
                    a[lane] = I::VOFF + row * 128 + I::vchunk(row, limb * 4 + 2 * c + hh) * 16;
                }
                CHECK(conflicts(a, 64, 16) == 1 && conflicts(a, 32, 8) == 1, "hd %d V read t %d c %d conflicts", HD, t,
                      c);
            }
    // the key order of a V row: the 8 positions 16c + 8hh + e hold keys 16c + 8(e/4) + 4hh + e%4
    for (int c = 0; c < 2; c++)
        for (int hh = 0; hh < 2; hh++)
            for (int e = 0; e < 8; e++)
                CHECK(I::vpos(16 * c + 8 * (e / 4) + 4 * hh + e % 4) == 16 * c + 8 * hh + e, "hd %d key order", HD);
    std::printf("hd %d: TB %d bytes, checked\n", HD, I::TB);
}

int main() {
    check<16>();
    check<24>();
    check<32>();
    check<64>();
    std::printf(fails ? "FAILED %d\n" : "OK\n", fails);
    return fails ? 1 : 0;
}
