// Host-side repacker check under AddressSanitizer and UndefinedBehaviorSanitizer (built and run by
// tests/test_host_sanitizers.py): every storage packed and unpacked at several shapes, row orders and group sizes, the
// dense bf16 round trip compared bit for bit, and one error path. Host code only; no GPU.
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>
#include <random>
#include "qwenny_hip.h"
static int check(int rc, const char* what) { if (rc < 0) { printf("%s: %d %s\n", what, rc, qh_last_error()); exit(1);} return rc; }
int main() {
    std::mt19937 rng(1);
    for (int bits : {4, 8}) for (int group : {128, 256, 0}) for (size_t rows : {16, 48, 96}) for (size_t cols : {128, 384, 1024}) {
        int g = group == 0 ? (int)cols : group;
        if (cols % g) continue;
        size_t words = cols * bits / 32, G = cols / g;
        std::vector<uint32_t> q(rows * words); for (auto& w : q) w = rng();
        if (bits == 8) for (auto& w : q) { uint32_t v = 0; for (int b = 0; b < 4; b++) { uint32_t x = 1 + rng() % 255; v |= x << (8*b);} w = v; }
        std::vector<float> sc(rows * G), off(rows * G);
        for (size_t i = 0; i < sc.size(); i++) { sc[i] = 0.01f * (1 + rng() % 7); off[i] = -(bits == 4 ? 8.f : 128.f) * sc[i]; }
        qh_quant Q{bits, g, rows, cols, q.data(), sc.data(), off.data()};
        std::vector<uint8_t> z(rows * G);
        check(qh_quant_zero_points(&Q, z.data()), "zp");
        int wt = bits == 8 ? QH_WT_I8 : QH_WT_I4;
        size_t cb, sb, zb; check(qh_packed_sizes(wt, rows, cols, &cb, &sb, &zb), "sizes");
        std::vector<uint8_t> codes(cb), scales(sb), zs(zb + 1);
        std::vector<size_t> order(rows); check(qh_row_order(rows, 1, order.data()), "order");
        check(qh_pack_quant(&Q, z.data(), order.data(), rows, wt, codes.data(), scales.data(), zs.data()), "pack");
        std::vector<uint8_t> vals(cols), zz(cols / 128); std::vector<float> s2(cols / 128);
        for (size_t p = 0; p < rows; p++) check(qh_unpack_row(wt, rows, cols, codes.data(), scales.data(), zs.data(), p, vals.data(), s2.data(), zz.data()), "unpack");
        std::vector<float> rowf(cols); for (size_t r = 0; r < rows; r++) check(qh_quant_row_into(&Q, r, rowf.data()), "row_into");
        // dense paths
        std::vector<uint16_t> w16(rows * cols); for (auto& v : w16) v = (uint16_t)(0x3c00 + rng() % 512);
        check(qh_packed_sizes(QH_WT_BF16, rows, cols, &cb, &sb, &zb), "sizes16");
        std::vector<uint8_t> c16(cb); check(qh_pack_dense_bf16(w16.data(), rows, cols, order.data(), rows, c16.data()), "pack16");
        std::vector<uint16_t> back(cols); for (size_t p = 0; p < rows; p++) { check(qh_unpack_row_bf16(rows, cols, c16.data(), p, back.data()), "unpack16"); if (memcmp(back.data(), &w16[order[p]*cols], cols*2)) { printf("bf16 mismatch\n"); return 1; } }
        check(qh_packed_sizes(QH_WT_I8, rows, cols, &cb, &sb, &zb), "sizes8");
        std::vector<uint8_t> c8(cb), s8(sb); check(qh_pack_dense_int8(w16.data(), rows, cols, order.data(), rows, c8.data(), s8.data()), "pack8");
    }
    // error paths
    qh_quant bad{4, 128, 16, 100, nullptr, nullptr, nullptr};
    if (qh_pack_quant(&bad, nullptr, nullptr, 16, QH_WT_I4, nullptr, nullptr, nullptr) >= 0) { printf("expected error\n"); return 1; }
    printf("asan driver ok\n");
    return 0;
}
