/*
 * AddressSanitizer / UndefinedBehaviorSanitizer run of the CPU oracle — TEST
 * INFRASTRUCTURE ONLY (built and run by `make -C oracle sanitize`, which
 * tests/test_sanitizers.py drives).
 *
 * Calls every orc_* function of rk_oracle.c on seeded random inputs and on
 * the edge cases the tests use (zero rows, FLT_MIN and huge values, ragged K,
 * odd packed widths, repeated experts, zero and negative routes, invalid
 * top-k), and checks relations that tie the functions together, so that the
 * sanitizers see every loop bound and index the tests rely on. Exit status 0
 * means no sanitizer report (the build aborts on the first one) and every
 * relation held.
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "rk_oracle.h"

static uint64_t rng = 0x5EED5EEDull;
static uint32_t next_u32(void) {
    rng = rng * 6364136223846793005ull + 1442695040888963407ull;
    return (uint32_t)(rng >> 33);
}
static float next_f(void) { return ((float)(next_u32() & 0xFFFFFF) / 16777216.0f) * 2.0f - 1.0f; }
static int8_t next_code(int bits) {
    return bits == 4 ? (int8_t)((int)(next_u32() % 16) - 8) : (int8_t)((int)(next_u32() % 255) - 127);
}

static int failures = 0;
#define CHECK(cond, ...)                  \
    do {                                  \
        if (!(cond)) {                    \
            fprintf(stderr, __VA_ARGS__); \
            fputc('\n', stderr);          \
            ++failures;                   \
        }                                 \
    } while (0)

static void* xmalloc(size_t n) {
    void* p = malloc(n ? n : 1);
    if (!p) {
        fprintf(stderr, "out of memory\n");
        exit(2);
    }
    return p;
}

static void check_quant(void) {
    const int ks[] = {1, 15, 16, 17, 63, 2560};
    for (size_t t = 0; t < sizeof(ks) / sizeof(ks[0]); ++t) {
        const int k = ks[t];
        float* x = xmalloc(sizeof(float) * k);
        int8_t* q = xmalloc(k);
        for (int row = 0; row < 5; ++row) {
            for (int i = 0; i < k; ++i) {
                const float v = next_f();
                x[i] = row == 0 ? 0.0f : row == 1 ? FLT_MIN * v : row == 2 ? 3e38f * v : row == 3 ? v * 20.0f : v;
            }
            float s_dense = 0.0f, s_moe = 0.0f;
            orc_quant_dense_row(x, k, q, &s_dense);
            for (int i = 0; i < k; ++i) CHECK(q[i] >= -127 && q[i] <= 127, "dense code out of range");
            CHECK(row != 0 || s_dense == 1.0f, "zero row scale %g", s_dense);
            CHECK(s_dense >= FLT_MIN, "dense scale below FLT_MIN");
            orc_quant_moe_row(x, k, q, &s_moe);
            for (int i = 0; i < k; ++i) CHECK(q[i] >= -127 && q[i] <= 127, "moe code out of range");
        }
        free(x);
        free(q);
    }
    for (int r = 0; r <= 300; ++r) {
        const int b = orc_bucket(r);
        if (r < 1 || r > 256)
            CHECK(b == -1, "bucket(%d) = %d outside 1..256", r, b);
        else
            CHECK(b >= r && b <= 256, "bucket(%d) = %d", r, b);
    }
}

static void check_linear(int bits) {
    const int k = 70, n = 64, rows = 3;
    int8_t* codes = xmalloc((size_t)k * n);
    float* scales = xmalloc(sizeof(float) * n);
    float* x = xmalloc(sizeof(float) * rows * k);
    float* y = xmalloc(sizeof(float) * rows * n);
    float* y2 = xmalloc(sizeof(float) * rows * n);
    int8_t* q = xmalloc((size_t)rows * k);
    float* s = xmalloc(sizeof(float) * rows);
    int32_t* acc = xmalloc(sizeof(int32_t) * rows * n);
    int32_t* acc2 = xmalloc(sizeof(int32_t) * rows * n);
    for (int i = 0; i < k * n; ++i) codes[i] = next_code(bits);
    for (int i = 0; i < n; ++i) scales[i] = 0.001f + 0.009f * fabsf(next_f());
    for (int i = 0; i < rows * k; ++i) x[i] = next_f() * 4.0f;
    orc_linear(codes, scales, k, n, x, rows, y, q, s, acc);
    orc_linear(codes, scales, k, n, x, rows, y2, NULL, NULL, NULL);
    CHECK(memcmp(y, y2, sizeof(float) * rows * n) == 0, "linear depends on the intermediates");
    orc_gemm_i8(q, codes, rows, k, n, acc2);
    CHECK(memcmp(acc, acc2, sizeof(int32_t) * rows * n) == 0, "linear accumulators differ from gemm");
    for (int r = 0; r < rows; ++r)
        for (int j = 0; j < n; ++j)
            CHECK(y[r * n + j] == orc_dequant(acc[r * n + j], s[r], scales[j]), "dequant relation");
    float* sw = xmalloc(sizeof(float) * rows * (n / 2));
    orc_linear_swiglu(codes, scales, k, n, x, rows, sw);
    for (int r = 0; r < rows; ++r)
        for (int j = 0; j < n / 2; ++j)
            CHECK(sw[r * (n / 2) + j] == orc_swiglu(y[r * n + j], y[r * n + n / 2 + j]), "swiglu relation");
    free(codes), free(scales), free(x), free(y), free(y2), free(q), free(s), free(acc), free(acc2), free(sw);
}

static void check_math(void) {
    for (int i = -800; i <= 800; ++i) {
        const float v = (float)i / 10.0f;
        const float e = orc_expf(v);
        CHECK(e > 0.0f && isfinite(e), "exp(%g) = %g", v, e);
    }
    const float edge[] = {-1e30f, -88.0f, -80.5f, -80.0f, -1.0f, -0.0f, 0.0f, 1.0f, 80.0f, 1e30f};
    for (size_t i = 0; i < sizeof(edge) / sizeof(edge[0]); ++i)
        for (size_t j = 0; j < sizeof(edge) / sizeof(edge[0]); ++j) (void)orc_swiglu(edge[i], edge[j]);
}

static void check_ffn(void) {
    const int h = 64, f = 96, rows = 2;
    int8_t* gc = xmalloc((size_t)h * 2 * f);
    float* gs = xmalloc(sizeof(float) * 2 * f);
    int8_t* dc = xmalloc((size_t)f * h);
    float* ds = xmalloc(sizeof(float) * h);
    float* x = xmalloc(sizeof(float) * rows * h);
    float* y = xmalloc(sizeof(float) * rows * h);
    float* mid = xmalloc(sizeof(float) * rows * f);
    float* mid2 = xmalloc(sizeof(float) * rows * f);
    float* y2 = xmalloc(sizeof(float) * rows * h);
    for (int i = 0; i < h * 2 * f; ++i) gc[i] = next_code(4);
    for (int i = 0; i < 2 * f; ++i) gs[i] = 0.001f + 0.009f * fabsf(next_f());
    for (int i = 0; i < f * h; ++i) dc[i] = next_code(8);
    for (int i = 0; i < h; ++i) ds[i] = 0.001f + 0.009f * fabsf(next_f());
    for (int i = 0; i < rows * h; ++i) x[i] = next_f();
    orc_ffn(gc, gs, dc, ds, h, f, x, rows, y, mid);
    orc_linear_swiglu(gc, gs, h, 2 * f, x, rows, mid2);
    CHECK(memcmp(mid, mid2, sizeof(float) * rows * f) == 0, "ffn middle differs from linear_swiglu");
    orc_linear(dc, ds, f, h, mid2, rows, y2, NULL, NULL, NULL);
    CHECK(memcmp(y, y2, sizeof(float) * rows * h) == 0, "ffn output differs from linear of the middle");
    free(gc), free(gs), free(dc), free(ds), free(x), free(y), free(mid), free(mid2), free(y2);
}

static void check_moe(void) {
    enum { E = 4, H = 32, I = 16, ROWS = 3, TOP = 2, SI = 24 };
    int8_t* gu[E];
    float* gus[E];
    int8_t* dn[E];
    float* dns[E];
    for (int e = 0; e < E; ++e) {
        gu[e] = xmalloc((size_t)H * 2 * I);
        gus[e] = xmalloc(sizeof(float) * 2 * I);
        dn[e] = xmalloc((size_t)I * H);
        dns[e] = xmalloc(sizeof(float) * H);
        for (int i = 0; i < H * 2 * I; ++i) gu[e][i] = next_code(4);
        for (int i = 0; i < 2 * I; ++i) gus[e][i] = 0.001f + 0.009f * fabsf(next_f());
        for (int i = 0; i < I * H; ++i) dn[e][i] = next_code(8);
        for (int i = 0; i < H; ++i) dns[e][i] = 0.001f + 0.009f * fabsf(next_f());
    }
    int8_t* sg = xmalloc((size_t)H * 2 * SI);
    float* sgs = xmalloc(sizeof(float) * 2 * SI);
    int8_t* sd = xmalloc((size_t)SI * H);
    float* sds = xmalloc(sizeof(float) * H);
    for (int i = 0; i < H * 2 * SI; ++i) sg[i] = next_code(8);
    for (int i = 0; i < 2 * SI; ++i) sgs[i] = 0.001f + 0.009f * fabsf(next_f());
    for (int i = 0; i < SI * H; ++i) sd[i] = next_code(8);
    for (int i = 0; i < H; ++i) sds[i] = 0.001f + 0.009f * fabsf(next_f());
    float x[ROWS * H];
    for (int i = 0; i < ROWS * H; ++i) x[i] = next_f();
    /* row 0: two experts; row 1: one expert twice; row 2: zero and negative routes */
    const int32_t ids[ROWS * TOP] = {1, 3, 2, 2, 0, 1};
    const float routes[ROWS * TOP] = {0.7f, 0.3f, 0.5f, 0.5f, 0.0f, -0.25f};
    float out[ROWS * H], out2[ROWS * H];
    orc_moe((const int8_t* const*)gu, (const float* const*)gus, (const int8_t* const*)dn,
            (const float* const*)dns, E, H, I, NULL, NULL, NULL, NULL, 0, x, ROWS, ids, routes, TOP, out);
    orc_moe((const int8_t* const*)gu, (const float* const*)gus, (const int8_t* const*)dn,
            (const float* const*)dns, E, H, I, sg, sgs, sd, sds, SI, x, ROWS, ids, routes, TOP, out2);
    for (int i = 0; i < H; ++i) CHECK(out[2 * H + i] == 0.0f, "skipped routes contributed");
    for (int e = 0; e < E; ++e) free(gu[e]), free(gus[e]), free(dn[e]), free(dns[e]);
    free(sg), free(sgs), free(sd), free(sds);
}

static void check_routes(void) {
    float logits[8];
    for (int i = 0; i < 8; ++i) logits[i] = next_f();
    logits[5] = logits[2]; /* a tie */
    int32_t ids[8];
    float w[8];
    CHECK(orc_routes(logits, 8, 3, ids, w) == 0, "routes rejected a valid top");
    float sum = 0.0f;
    for (int i = 0; i < 3; ++i) sum += w[i];
    CHECK(fabsf(sum - 1.0f) < 1e-5f, "route weights sum to %g", sum);
    CHECK(orc_routes(logits, 8, 0, ids, w) != 0, "routes accepted top 0");
    CHECK(orc_routes(logits, 8, 9, ids, w) != 0, "routes accepted top > count");
}

static void check_unpack(void) {
    const int bitss[] = {4, 8};
    for (int b = 0; b < 2; ++b) {
        const int bits = bitss[b], n = 5, k = 37;
        const int wpr = (k * bits + 31) / 32;
        uint32_t* words = xmalloc(sizeof(uint32_t) * n * wpr);
        for (int i = 0; i < n * wpr; ++i) words[i] = next_u32();
        int8_t* codes = xmalloc((size_t)k * n);
        orc_unpack_codes(words, bits, n, k, codes);
        for (int i = 0; i < k * n; ++i)
            CHECK(bits == 8 || (codes[i] >= -8 && codes[i] <= 7), "W4 code out of range");
        free(words), free(codes);
    }
    int8_t a[3 * 2], bb[3 * 5];
    for (int i = 0; i < 6; ++i) a[i] = (int8_t)i;
    for (int i = 0; i < 15; ++i) bb[i] = (int8_t)(100 + i);
    const int8_t* parts[2] = {a, bb};
    const int ns[2] = {2, 5};
    int8_t out[3 * 7];
    orc_concatenate(parts, ns, 2, 3, out);
    for (int r = 0; r < 3; ++r) {
        CHECK(out[r * 7 + 0] == a[r * 2 + 0] && out[r * 7 + 1] == a[r * 2 + 1], "concatenate, first part");
        for (int j = 0; j < 5; ++j) CHECK(out[r * 7 + 2 + j] == bb[r * 5 + j], "concatenate, second part");
    }
}

int main(void) {
    check_quant();
    check_linear(4);
    check_linear(8);
    check_math();
    check_ffn();
    check_moe();
    check_routes();
    check_unpack();
    printf("oracle sanitizer run: %d failed checks, threads %d\n", failures, orc_threads());
    return failures == 0 ? 0 : 1;
}
