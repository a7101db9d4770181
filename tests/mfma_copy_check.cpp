// Host check of the direct-to-LDS copy plan of mfma_gemm
// (tau.rs_amd/csrc/mfma_copy_plan.hpp), for every compiled tile and the
// prefill shapes of the benchmark configurations:
//  * the two-word scalar address round trip keeps addresses whose low word
//    has bit 31 set (the sign-extension fault of the 128x128 wave tiles);
//  * one stage's copies write every LDS chunk of the A and B panels exactly
//    once, and each staged row receives every K chunk of its source row once;
//  * every per-lane source offset, advanced to the last K step, stays inside
//    its tensor (A: the activations or the gathered x rows; B: one expert's
//    weights) and fits the 32-bit per-lane offsets of the 128x128 wave tiles.
// Prints "ok <checks>" and exits 0, or prints the first violation and exits 1.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include <vector>

#include "../tau.rs_amd/csrc/mfma_copy_plan.hpp"

using namespace tau_amd;

static long checks = 0;

#define REQUIRE(cond, ...)                      \
    do {                                        \
        ++checks;                               \
        if (!(cond)) {                          \
            printf("FAIL %s: ", #cond);         \
            printf(__VA_ARGS__);                \
            printf("\n");                       \
            exit(1);                            \
        }                                       \
    } while (0)

static long capacity(long T, long E, long K, long M) {
    const long a = T * K;
    return (a + (a < E ? a : E) * (M - 1) + (M - 1)) / M * M;
}

struct Shape {
    const char* name;
    int T, H, I, E, K;
};

// One tile configuration and projection: BM x BN tile, NT threads, BK = 64.
template <int BM, int BN, int WM, int WN, bool SILU, bool FRAG16>
static void check_tile(const Shape& s) {
    constexpr int BK = 64, CPR = BK / 8, NT = 64 * WM * WN;
    constexpr int ACH = BM * CPR / NT, BCH = BN * CPR / NT;
    static_assert(ACH * NT == BM * CPR && BCH * NT == BN * CPR, "tile/threads");
    // gate_up (SILU): A = x [T, H] gathered, K = H, n = I, weights [2I, H].
    // down: A = activated [cap, I] direct, K = I, n = H, weights [H, I].
    const long cap = capacity(s.T, s.E, s.K, BM);
    const long a_rows = SILU ? s.T : cap;
    const int k = SILU ? s.H : s.I, lda = k;
    const int n = SILU ? s.I : s.H;
    const long w_rows = SILU ? 2L * s.I : s.H;
    const long expert_elems = w_rows * k;
    const int w_up = SILU ? s.I : 0;
    const long a_bytes = a_rows * lda * 2;

    // A stage coverage and bounds.
    std::vector<int> lds_hits(BM * CPR, 0), src_hits(BM * CPR, 0);
    for (int w = 0; w < NT / 64; ++w)
        for (int i = 0; i < ACH; ++i)
            for (int lane = 0; lane < 64; ++lane) {
                int r, kchunk;
                row_copy_slot<NT, CPR>(i, w, lane, r, kchunk);
                REQUIRE(r >= 0 && r < BM, "%s A row %d", s.name, r);
                REQUIRE(kchunk % 8 == 0 && kchunk >= 0 && kchunk < BK, "%s A kchunk %d", s.name, kchunk);
                // LDS destination: instruction (i, w) fills 1 KB at (i*(NT/64)+w)*512 elements.
                const int lds_chunk = (i * (NT / 64) + w) * 64 + lane;
                REQUIRE(lds_chunk / CPR == r && lds_chunk % CPR == (lane % CPR), "%s A LDS slot", s.name);
                ++lds_hits[lds_chunk];
                ++src_hits[r * CPR + kchunk / 8];
                // the last source row of A at the last K step, 16 bytes read
                const long off = ((a_rows - 1) * (long)lda + kchunk + (k - BK)) * 2;
                REQUIRE(off >= 0 && off + 16 <= a_bytes, "%s A offset %ld of %ld", s.name, off, a_bytes);
                REQUIRE(off < (1L << 32), "%s A offset %ld exceeds 32 bits", s.name, off);
            }
    for (int c = 0; c < BM * CPR; ++c) {
        REQUIRE(lds_hits[c] == 1, "%s A LDS chunk %d written %d times", s.name, c, lds_hits[c]);
        REQUIRE(src_hits[c] == 1, "%s A source chunk %d read %d times", s.name, c, src_hits[c]);
    }

    // B stage coverage and bounds, for every output tile column.
    const int nout = SILU ? BN / 2 : BN;
    for (int c0 = 0; c0 < n; c0 += nout) {
        std::vector<int> hits(BN * CPR, 0);
        for (int w = 0; w < NT / 64; ++w)
            for (int i = 0; i < BCH; ++i)
                for (int lane = 0; lane < 64; ++lane) {
                    const long off = b_copy_offset<NT, CPR, BN, BK, SILU, FRAG16>(i, w, lane, c0, n, w_up, k);
                    const long last = FRAG16 ? off + (long)(k - BK) * 16 : off + (k - BK);
                    REQUIRE(off >= 0 && last + 8 <= expert_elems, "%s B offset %ld of %ld (c0 %d)", s.name, last,
                            expert_elems, c0);
                    REQUIRE(last * 2 < (1L << 32), "%s B offset exceeds 32 bits", s.name);
                    const int q = i * (NT / 64) + w;
                    if (FRAG16) {
                        // fragment q of the stage: 16 rows x 32 K; lane = 16-byte piece
                        REQUIRE(q < BN / 16 * (BK / 32), "%s B fragment %d", s.name, q);
                        ++hits[q * 64 + lane];
                        // the fragment's band and K piece: rows 16*band.. of the tile
                        const int band = q / (BK / 32), kp = q % (BK / 32);
                        const long row = weight_row<BN, SILU>(band * 16, c0, n, w_up);
                        REQUIRE(row % 16 == 0, "%s B band row %ld", s.name, row);
                        REQUIRE(off == (row / 16) * 16L * k + kp * 512 + lane * 8, "%s B frag16 offset", s.name);
                    } else {
                        int r, kchunk;
                        row_copy_slot<NT, CPR>(i, w, lane, r, kchunk);
                        REQUIRE(r < BN, "%s B row %d", s.name, r);
                        ++hits[r * CPR + kchunk / 8];
                        const long row = weight_row<BN, SILU>(r, c0, n, w_up);
                        REQUIRE(off == row * k + kchunk, "%s B row-major offset", s.name);
                    }
                }
        for (int c = 0; c < BN * CPR; ++c) REQUIRE(hits[c] == 1, "%s B chunk %d hit %d times", s.name, c, hits[c]);
    }
    // SiLU tiles pair gate row j with up row j + I.
    if (SILU)
        for (int r = 0; r < BN / 2; ++r) {
            const long g = weight_row<BN, true>(r, 0, n, w_up), u = weight_row<BN, true>(r + BN / 2, 0, n, w_up);
            if (r < n) REQUIRE(u == g + s.I, "%s gate/up pairing", s.name);
        }
}

template <int BM, int BN, int WM, int WN>
static void check_config(const Shape& s) {
    check_tile<BM, BN, WM, WN, true, true>(s);
    check_tile<BM, BN, WM, WN, true, false>(s);
    check_tile<BM, BN, WM, WN, false, true>(s);
    check_tile<BM, BN, WM, WN, false, false>(s);
}

int main() {
    // Addresses whose low word has bit 31 set survive the two-word round trip.
    const uint64_t addrs[] = {0x00007f1280001000ull, 0x00007fffffffff00ull, 0x0000000080000000ull,
                              0x00007f12000010f0ull};
    for (uint64_t a : addrs) {
        REQUIRE(join_address(address_hi(a), address_lo(a)) == a, "round trip of %llx", (unsigned long long)a);
        // the faulty composition: the low word through int, sign-extended
        const uint64_t bad = ((uint64_t)address_hi(a) << 32) | (uint64_t)(int64_t)(int32_t)address_lo(a);
        if (address_lo(a) & 0x80000000u) REQUIRE(bad != a, "sign extension not exercised");
    }
    const Shape shapes[] = {
        {"c3", 4096, 2048, 768, 128, 8},  {"c5p", 8192, 4096, 1536, 128, 8}, {"c4", 2048, 2048, 512, 513, 11},
        {"c3_t1024", 1024, 2048, 768, 128, 8}, {"odd", 37, 256, 192, 24, 3},
    };
    for (const Shape& s : shapes) {
        check_config<256, 256, 4, 4>(s);  // shipped 256-row tile
        check_config<256, 256, 2, 2>(s);  // 128x128 wave tiles (-DTAU_M256_BIG_WAVES)
        check_config<128, 128, 2, 2>(s);
        check_config<64, 256, 1, 4>(s);
    }
    printf("ok %ld\n", checks);
    return 0;
}
