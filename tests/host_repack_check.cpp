// Host repack round trips, built alone under AddressSanitizer + UndefinedBehaviorSanitizer (and ThreadSanitizer) by
// tests/test_host_sanitizers.py: every buffer is allocated at its exact size, so a read or write one byte past a
// plane or a row is reported. For each GGUF type, every GGUF type in 16-row tiles and the tiled int8 planes, at shapes that run
// on one host thread and on several:
//   * repack into a buffer full of 0xAB, unpack, and compare with the input bytes;
//   * the alignment padding between planes (and the int8 tiles' padding rows and columns) reads zero;
//   * the planes are the same bytes on 1 thread and on 5 (written into buffers of different filler bytes: so every
//     byte is written, the tiles' padding rows included).
#include <stdint.h>
#include <stdio.h>

#include <vector>

#include "mbq_host_repack.h"

using namespace mbq;

static uint64_t g_state = 0x9E3779B97F4A7C15ull;
static uint8_t rnd8() {
    g_state ^= g_state << 13;
    g_state ^= g_state >> 7;
    g_state ^= g_state << 17;
    return (uint8_t)(g_state >> 24);
}

static int g_fail = 0;
#define CHECK(cond, ...)                   \
    do {                                   \
        if (!(cond)) {                     \
            fprintf(stderr, __VA_ARGS__);  \
            fprintf(stderr, "\n");         \
            ++g_fail;                      \
        }                                  \
    } while (0)

static void gguf_case(int t, int64_t rows, int64_t cols) {
    const int64_t rb = cols / block_values(t) * block_bytes(t);
    const Layout L = layout(t, rows, cols);
    std::vector<uint8_t> raw((size_t)(rows * rb)), back((size_t)(rows * rb), 0x5A);
    for (auto& b : raw) b = rnd8();
    std::vector<uint8_t> p1((size_t)L.total, 0xAB), p5((size_t)L.total, 0xCD);
    repack_host(t, raw.data(), rows, cols, p1.data(), 1);
    repack_host(t, raw.data(), rows, cols, p5.data(), 5);
    CHECK(p1 == p5, "type %d (%lld, %lld): planes differ between 1 and 5 threads", t, (long long)rows, (long long)cols);
    for_each_gap(L, [&](int64_t off, int64_t n) {
        for (int64_t i = 0; i < n; ++i)
            if (p1[(size_t)(off + i)] != 0) {
                CHECK(false, "type %d (%lld, %lld): padding byte %lld is not zero", t, (long long)rows, (long long)cols,
                      (long long)(off + i));
                return false;
            }
        return true;
    });
    unpack_host(t, p1.data(), rows, cols, back.data(), 3);
    CHECK(back == raw, "type %d (%lld, %lld): unpack(repack(raw)) != raw", t, (long long)rows, (long long)cols);
}

static void int8_case(int64_t rows, int64_t cols) {
    const Layout L = layout(T_I8T, rows, cols);
    std::vector<int8_t> q((size_t)(rows * cols)), q2((size_t)(rows * cols), 7);
    std::vector<float> s((size_t)rows), s2((size_t)rows, -1.f);
    for (auto& v : q) v = (int8_t)rnd8();
    for (int64_t i = 0; i < rows; ++i) s[(size_t)i] = 1e-3f * (float)(1 + (rnd8() % 9));
    std::vector<uint8_t> p1((size_t)L.total, 0xAB), p5((size_t)L.total, 0xCD);
    i8t_repack_host(q.data(), s.data(), rows, cols, p1.data(), 1);
    i8t_repack_host(q.data(), s.data(), rows, cols, p5.data(), 5);
    CHECK(p1 == p5, "int8 (%lld, %lld): planes differ between 1 and 5 threads", (long long)rows, (long long)cols);
    // padding rows and columns of every tile, and the scales of padding rows, are zero
    const int64_t kc_n = (cols + 63) / 64, np = (rows + 15) / 16 * 16;
    for (int64_t row = 0; row < np; ++row)
        for (int64_t k = 0; k < kc_n * 64; ++k) {
            if (row < rows && k < cols) continue;
            const uint8_t v = p1[(size_t)(L.qs_off + i8t_off(row, cols, k & ~int64_t(63)) + (k & 63))];
            CHECK(v == 0, "int8 (%lld, %lld): padding value (%lld, %lld) = %d", (long long)rows, (long long)cols,
                  (long long)row, (long long)k, v);
        }
    for (int64_t row = rows; row < np; ++row) {
        float v;
        memcpy(&v, &p1[(size_t)(L.sc_off + row * 4)], 4);
        CHECK(v == 0.f, "int8 (%lld, %lld): padding row %lld has scale %g", (long long)rows, (long long)cols, (long long)row, v);
    }
    for_each_gap(L, [&](int64_t off, int64_t n) {
        for (int64_t i = 0; i < n; ++i) CHECK(p1[(size_t)(off + i)] == 0, "int8 (%lld, %lld): gap byte not zero", (long long)rows, (long long)cols);
        return true;
    });
    i8t_unpack_host(p1.data(), rows, cols, q2.data(), s2.data(), 3);
    CHECK(q2 == q && s2 == s, "int8 (%lld, %lld): unpack(repack(q, s)) != (q, s)", (long long)rows, (long long)cols);
}

int main() {
    const int types[] = {T_Q4_0, T_Q8_0, T_Q4_K, T_Q5_K, T_Q6_K, T_Q4KT, T_Q8T, T_Q6KT, T_Q5KT, T_Q40T};
    const int64_t shapes[][2] = {{1, 256}, {3, 512}, {63, 768}, {64, 256}, {130, 1024}, {517, 256}};
    for (int t : types)
        for (const auto& sh : shapes) gguf_case(t, sh[0], sh[1]);
    for (int64_t c : {32, 96}) gguf_case(T_Q8_0, 200, c), gguf_case(T_Q8T, 200, c), gguf_case(T_Q4_0, 200, c), gguf_case(T_Q40T, 200, c);
    const int64_t i8[][2] = {{1, 16}, {15, 48}, {16, 64}, {17, 80}, {100, 4112}, {1040, 128}, {33, 1000 * 16}};
    for (const auto& sh : i8) int8_case(sh[0], sh[1]);
    if (g_fail) {
        fprintf(stderr, "%d check(s) failed\n", g_fail);
        return 1;
    }
    printf("host repack round trips ok\n");
    return 0;
}
