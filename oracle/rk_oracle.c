/*
 * CPU oracle for the quantized-linear hot path — TEST INFRASTRUCTURE ONLY.
 * See rk_oracle.h. Built with -ffp-contract=off so every float operation is
 * the single IEEE operation written here (no fused multiply-add unless fmaf()
 * is written explicitly).
 */
#include "rk_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int orc_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* src/npu.rs:201-211: 1..=256 rows; <=128 -> next power of two, else a
 * multiple of 64. Returns -1 outside the legal range. */
int orc_bucket(int rows) {
    if (rows < 1 || rows > 256) return -1;
    if (rows <= 128) {
        int m = 1;
        while (m < rows) m <<= 1;
        return m;
    }
    return (rows + 63) / 64 * 64;
}

static float row_maxabs(const float* x, int k) {
    /* src/npu.rs:1539: fold(0.0, |m, x| m.max(x.abs())) */
    float m = 0.0f;
    for (int i = 0; i < k; ++i) m = fmaxf(m, fabsf(x[i]));
    return m;
}

/* src/npu.rs:1537-1547:
 *   scale = max == 0 ? 1 : max(max / 127, FLT_MIN)
 *   q     = clamp(round_half_away(x * (1 / scale)), -127, 127)  */
void orc_quant_dense_row(const float* x, int k, int8_t* codes, float* scale) {
    float m = row_maxabs(x, k);
    float s = (m == 0.0f) ? 1.0f : fmaxf(m / 127.0f, FLT_MIN);
    float inv = 1.0f / s;
    for (int i = 0; i < k; ++i) {
        float v = roundf(x[i] * inv);
        if (v < -127.0f) v = -127.0f;
        if (v > 127.0f) v = 127.0f;
        codes[i] = (int8_t)v;
    }
    *scale = s;
}

/* MOE_CPU_FUSION_20261023.md:13: the MoE path keeps nearest-even rounding,
 * an all-zero row gets scale 1, and there is no FLT_MIN floor. */
void orc_quant_moe_row(const float* x, int k, int8_t* codes, float* scale) {
    float m = row_maxabs(x, k);
    float s = (m == 0.0f) ? 1.0f : m / 127.0f;
    float inv = 1.0f / s;
    for (int i = 0; i < k; ++i) {
        float v = rintf(x[i] * inv);
        if (v < -127.0f) v = -127.0f;
        if (v > 127.0f) v = 127.0f;
        codes[i] = (int8_t)v;
    }
    *scale = s;
}

/* src/npu.rs:1548-1552: exact int32 dot over K, w laid out [K][N]. Row blocks
 * of 4 and column blocks of 256 keep the weight panel in cache. */
void orc_gemm_i8(const int8_t* a, const int8_t* w, int m, int k, int n, int32_t* acc) {
    enum { RB = 4, CB = 256 };
    int row_blocks = (m + RB - 1) / RB;
    int col_blocks = (n + CB - 1) / CB;
#pragma omp parallel for schedule(dynamic) collapse(2)
    for (int rb = 0; rb < row_blocks; ++rb) {
        for (int cb = 0; cb < col_blocks; ++cb) {
            int32_t local[RB][CB];
            int r0 = rb * RB, c0 = cb * CB;
            int rows = m - r0 < RB ? m - r0 : RB;
            int cols = n - c0 < CB ? n - c0 : CB;
            memset(local, 0, sizeof(local));
            for (int kk = 0; kk < k; ++kk) {
                const int8_t* wr = w + (size_t)kk * n + c0;
                for (int r = 0; r < rows; ++r) {
                    int32_t av = a[(size_t)(r0 + r) * k + kk];
                    if (av == 0) continue;
                    int32_t* lr = local[r];
                    for (int c = 0; c < cols; ++c) lr[c] += av * (int32_t)wr[c];
                }
            }
            for (int r = 0; r < rows; ++r)
                memcpy(acc + (size_t)(r0 + r) * n + c0, local[r], (size_t)cols * sizeof(int32_t));
        }
    }
}

/* src/npu.rs:1553: (sum as f32 * scale) * scales[n] — two RNE multiplies. */
float orc_dequant(int32_t acc, float row_scale, float col_scale) {
    float y = (float)acc * row_scale;
    return y * col_scale;
}

void orc_linear(const int8_t* codes, const float* scales, int k, int n,
                const float* input, int rows, float* output,
                int8_t* q_out, float* s_out, int32_t* acc_out) {
    int8_t* q = q_out ? q_out : (int8_t*)malloc((size_t)rows * k);
    float* s = s_out ? s_out : (float*)malloc((size_t)rows * sizeof(float));
    int32_t* acc = acc_out ? acc_out : (int32_t*)malloc((size_t)rows * n * sizeof(int32_t));
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) orc_quant_dense_row(input + (size_t)r * k, k, q + (size_t)r * k, s + r);
    orc_gemm_i8(q, codes, rows, k, n, acc);
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r)
        for (int c = 0; c < n; ++c)
            output[(size_t)r * n + c] = orc_dequant(acc[(size_t)r * n + c], s[r], scales[c]);
    if (!q_out) free(q);
    if (!s_out) free(s);
    if (!acc_out) free(acc);
}

/* exp(x) for |x| <= 80, written from Cody and Waite's additive range
 * reduction: x = n*ln2 + r with n = rint(x*log2(e)) and ln2 split into a
 * 12-bit-short high part and a low part; e^r from its degree-7 Taylor series
 * (coefficients 1/j!, rounded to f32) in Horner form; 2^n applied through the
 * exponent field (n stays within [-116, 116], so 2^n is a normal float).
 * Every step is one IEEE operation, so CPU and GPU evaluate identical bits. */
float orc_expf(float x) {
    const float log2e = 0x1.715476p+0f;
    const float ln2_hi = 0x1.62ep-1f;
    const float ln2_lo = 0x1.0bfbe8p-15f;
    float kf = rintf(x * log2e);
    float r = fmaf(kf, -ln2_hi, x);
    r = fmaf(kf, -ln2_lo, r);
    float p = 0x1.a01a02p-13f;            /* 1/7! */
    p = fmaf(p, r, 0x1.6c16c2p-10f);      /* 1/6! */
    p = fmaf(p, r, 0x1.111112p-7f);       /* 1/5! */
    p = fmaf(p, r, 0x1.555556p-5f);       /* 1/4! */
    p = fmaf(p, r, 0x1.555556p-3f);       /* 1/3! */
    p = fmaf(p, r, 0x1.0p-1f);            /* 1/2! */
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    int n = (int)kf;
    uint32_t bits = (uint32_t)(n + 127) << 23;
    float two_n;
    memcpy(&two_n, &bits, sizeof(two_n));
    return p * two_n;
}

/* silu(g) * u = (g / (1 + exp(-g))) * u. The exponent argument saturates to
 * [-80, 80] and a gate below -80 yields a signed zero, the range handling of
 * the reference's fused FP32 activation. */
float orc_swiglu(float gate, float up) {
    float t = -gate;
    if (t < -80.0f) t = -80.0f;
    if (t > 80.0f) t = 80.0f;
    float e = orc_expf(t);
    float silu = gate / (1.0f + e);
    if (gate < -80.0f) silu = copysignf(0.0f, gate);
    return silu * up;
}

void orc_linear_swiglu(const int8_t* codes, const float* scales, int k, int n,
                       const float* input, int rows, float* output) {
    int half = n / 2;
    float* y = (float*)malloc((size_t)rows * n * sizeof(float));
    orc_linear(codes, scales, k, n, input, rows, y, NULL, NULL, NULL);
    for (int r = 0; r < rows; ++r)
        for (int j = 0; j < half; ++j)
            output[(size_t)r * half + j] = orc_swiglu(y[(size_t)r * n + j], y[(size_t)r * n + half + j]);
    free(y);
}

void orc_ffn(const int8_t* gu_codes, const float* gu_scales,
             const int8_t* dn_codes, const float* dn_scales, int h, int f,
             const float* input, int rows, float* output, float* mid_out) {
    float* mid = mid_out ? mid_out : (float*)malloc((size_t)rows * f * sizeof(float));
    orc_linear_swiglu(gu_codes, gu_scales, h, 2 * f, input, rows, mid);
    /* The middle is requantized with the dense rule over the whole row. */
    orc_linear(dn_codes, dn_scales, f, h, mid, rows, output, NULL, NULL, NULL);
    if (!mid_out) free(mid);
}

/* One expert FFN on one MoE-quantized row: gate/up GEMM, dequant, SwiGLU,
 * nearest-even requant of the (token, expert) middle row, down GEMM,
 * dequant into contrib[h]. */
static void moe_expert_row(const int8_t* q, float s, int h, int inter,
                           const int8_t* gu, const float* gus,
                           const int8_t* dn, const float* dns,
                           int32_t* acc_gu, float* mid, int8_t* qm, int32_t* acc_dn,
                           float* contrib) {
    orc_gemm_i8(q, gu, 1, h, 2 * inter, acc_gu);
    for (int j = 0; j < inter; ++j) {
        float g = orc_dequant(acc_gu[j], s, gus[j]);
        float u = orc_dequant(acc_gu[inter + j], s, gus[inter + j]);
        mid[j] = orc_swiglu(g, u);
    }
    float sm;
    orc_quant_moe_row(mid, inter, qm, &sm);
    orc_gemm_i8(qm, dn, 1, inter, h, acc_dn);
    for (int c = 0; c < h; ++c) contrib[c] = orc_dequant(acc_dn[c], sm, dns[c]);
}

void orc_moe(const int8_t* const* gu_codes, const float* const* gu_scales,
             const int8_t* const* dn_codes, const float* const* dn_scales,
             int experts, int h, int inter,
             const int8_t* sh_gu_codes, const float* sh_gu_scales,
             const int8_t* sh_dn_codes, const float* sh_dn_scales, int sh_inter,
             const float* input, int rows, const int32_t* ids, const float* routes,
             int top, float* output) {
    (void)experts;
    int wide = inter > sh_inter ? inter : sh_inter;
#pragma omp parallel for schedule(dynamic)
    for (int r = 0; r < rows; ++r) {
        int8_t* q = (int8_t*)malloc((size_t)h);
        int32_t* acc_gu = (int32_t*)malloc((size_t)2 * wide * sizeof(int32_t));
        float* mid = (float*)malloc((size_t)wide * sizeof(float));
        int8_t* qm = (int8_t*)malloc((size_t)wide);
        int32_t* acc_dn = (int32_t*)malloc((size_t)h * sizeof(int32_t));
        float* contrib = (float*)malloc((size_t)h * sizeof(float));
        float* sum = output + (size_t)r * h;
        float s;
        /* The token row is quantized once and shared by all its experts. */
        orc_quant_moe_row(input + (size_t)r * h, h, q, &s);
        for (int c = 0; c < h; ++c) sum[c] = 0.0f;
        for (int rank = 0; rank < top; ++rank) {
            float route = routes[(size_t)r * top + rank];
            /* src/model/experts/paged.rs:500-504: skipped entries (route <= 0)
             * contribute nothing; the rest accumulate in rank order with fma. */
            if (!(route > 0.0f)) continue;
            int e = ids[(size_t)r * top + rank];
            moe_expert_row(q, s, h, inter, gu_codes[e], gu_scales[e], dn_codes[e], dn_scales[e],
                           acc_gu, mid, qm, acc_dn, contrib);
            for (int c = 0; c < h; ++c) sum[c] = fmaf(contrib[c], route, sum[c]);
        }
        if (sh_gu_codes) {
            /* MOE_ROUTED_SHARED_JOINT_20261023.md:19: the shared expert is
             * added after the routed sum. */
            moe_expert_row(q, s, h, sh_inter, sh_gu_codes, sh_gu_scales, sh_dn_codes, sh_dn_scales,
                           acc_gu, mid, qm, acc_dn, contrib);
            for (int c = 0; c < h; ++c) sum[c] = sum[c] + contrib[c];
        }
        free(q); free(acc_gu); free(mid); free(qm); free(acc_dn); free(contrib);
    }
}

/* f32::total_cmp key: flips the magnitude bits of negatives so that signed
 * integer order equals the IEEE total order (-0.0 < +0.0). */
static int32_t total_key(float v) {
    int32_t b;
    memcpy(&b, &v, sizeof(b));
    return b ^ (int32_t)(((uint32_t)(b >> 31)) >> 1);
}

int orc_routes(const float* logits, int count, int top, int32_t* ids, float* weights) {
    if (top <= 0 || top > count) return -1;
    /* Selection by repeated maximum keeps the comparator of
     * src/model/qwen35/moe.rs:58 (descending total order, lower id first). */
    char* taken = (char*)calloc((size_t)count, 1);
    for (int t = 0; t < top; ++t) {
        int best = -1;
        for (int i = 0; i < count; ++i) {
            if (taken[i]) continue;
            if (best < 0 || total_key(logits[i]) > total_key(logits[best])) best = i;
        }
        taken[best] = 1;
        ids[t] = best;
    }
    free(taken);
    float max = logits[ids[0]];
    float sum = 0.0f;
    for (int t = 0; t < top; ++t) {
        weights[t] = expf(logits[ids[t]] - max);
        sum += weights[t];
    }
    for (int t = 0; t < top; ++t) weights[t] /= sum;
    return 0;
}

void orc_unpack_codes(const uint32_t* words, int bits, int n, int k, int8_t* codes) {
    int factor = 32 / bits;
    int columns = (k + factor - 1) / factor;
    uint32_t mask = (bits == 32) ? 0xffffffffu : ((1u << bits) - 1u);
    for (int ki = 0; ki < k; ++ki)
        for (int ni = 0; ni < n; ++ni) {
            uint32_t word = words[(size_t)ni * columns + ki / factor];
            int32_t v = (int32_t)((word >> ((ki % factor) * bits)) & mask) - (1 << (bits - 1));
            codes[(size_t)ki * n + ni] = (int8_t)v;
        }
}

void orc_concatenate(const int8_t* const* codes, const int* ns, int count, int k, int8_t* out) {
    int n = 0;
    for (int i = 0; i < count; ++i) n += ns[i];
    for (int ki = 0; ki < k; ++ki) {
        int offset = 0;
        for (int i = 0; i < count; ++i) {
            memcpy(out + (size_t)ki * n + offset, codes[i] + (size_t)ki * ns[i], (size_t)ns[i]);
            offset += ns[i];
        }
    }
}

/* Steele, Lea and Flood's SplitMix64 generator. */
uint64_t orc_splitmix64(uint64_t* state) {
    uint64_t z = (*state += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
