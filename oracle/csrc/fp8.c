/*
 * CPU oracle for the e4m3 expert variant. TEST INFRASTRUCTURE ONLY (tests/, __graft_entry__.smoke(), bench.py's
 * CPU-baseline leg); the shipped library never links it.
 *
 * Numerics (the reference's e4m3 contract, code/fork/kernels/moe_e4m3.cu:1-25, code/fork/overlay/glm53_moe_e4m3.py:
 * 648-674, applied to block-scaled e4m3 experts):
 *   e4m3      OCP float8 E4M3FN: bias 7, 3 mantissa bits, max 448, no infinities; round to nearest even
 *   quant     per row: s = amax(|v|) / 448 (1 if 0), q = e4m3(clamp(v / s, -448, 448))     (moe_e4m3.cu:152-176)
 *   gate/up   acc = sum over 128-k blocks b of ws[n/128][b] * (sum_{k in b} q_x[k] * W8[n][k]); g = acc * s_x
 *   act       a16 = fp16(silu(min(g, L)) * clamp(u, -L, L)) (limit iff L != 0), silu(v) = v / (1 + exp(-v))
 *   down      the same GEMM over q_a = quant(a16 row) with the down block scales; out[token] += w * acc * s_a
 * mode 0 evaluates the sums in fp32 in k order per 128-block (the kernels' rounding points up to the order inside
 * a block); mode 1 evaluates every sum and the activation in float64 from the same quantized operands.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

float orc_h2f(uint16_t h);
uint16_t orc_f2h(float f);
uint16_t orc_d2h(double d);

/* ---------------------------------------------------------------- e4m3 */

uint8_t orc_e4m3_from_f32(float f) {
    if (isnan(f)) return 0x7F;
    const uint8_t sign = signbit(f) ? 0x80 : 0x00;
    const double a = fabs((double)f);
    if (a >= 448.0) return sign | 0x7E;                             /* saturate (callers clamp first) */
    if (a < ldexp(1.0, -6)) {                                        /* subnormal range: multiples of 2^-9 */
        const double q = nearbyint(a * 512.0);                       /* RN-even; q = 8 is the smallest normal */
        return sign | (uint8_t)q;
    }
    int ex;
    const double fr = frexp(a, &ex);                                 /* a = fr * 2^ex, fr in [0.5, 1) */
    int E = ex - 1;                                                  /* a = m * 2^E, m in [1, 2) */
    double m = nearbyint((ldexp(fr, 1) - 1.0) * 8.0);                /* 3 mantissa bits, RN-even */
    if (m == 8.0) {
        m = 0.0;
        ++E;
    }
    int code = ((E + 7) << 3) | (int)m;
    if (code > 0x7E) code = 0x7E;
    return sign | (uint8_t)code;
}

float orc_e4m3_to_f32(uint8_t b) {
    if ((b & 0x7F) == 0x7F) return NAN;
    const int E = (b >> 3) & 15, m = b & 7;
    const double v = E == 0 ? ldexp((double)m, -9) : ldexp(1.0 + m / 8.0, E - 7);
    return (float)((b & 0x80) ? -v : v);
}

/* per row: s = amax / 448 (1 if 0), q = e4m3(clamp(v / s)); fp32 division as written */
void orc_quant_rows(const float* x, int rows, int K, uint8_t* q, float* s) {
    for (int r = 0; r < rows; ++r) {
        const float* v = x + (size_t)r * K;
        float amax = 0.0f;
        for (int k = 0; k < K; ++k) amax = fmaxf(amax, fabsf(v[k]));
        float sc = amax / 448.0f;
        if (!(sc > 0.0f)) sc = 1.0f;
        s[r] = sc;
        for (int k = 0; k < K; ++k) {
            float t = v[k] / sc;
            t = fminf(fmaxf(t, -448.0f), 448.0f);
            q[(size_t)r * K + k] = orc_e4m3_from_f32(t);
        }
    }
}

/* ---------------------------------------------------------------- block-scaled e4m3 experts */

typedef struct {
    int n, K, N;
    const uint8_t* w13;      /* [n][2N][K]  rows 0..N-1 gate, N..2N-1 up */
    const float* w13s;       /* [n][2N/128][K/128] */
    const uint8_t* w2;       /* [n][K][N] */
    const float* w2s;        /* [n][K/128][N/128] */
} orc_fp8_layer;

static float g_e4[256];
static int g_e4_ready = 0;
static void e4_init(void) {
    if (g_e4_ready) return;
    for (int b = 0; b < 256; ++b) g_e4[b] = orc_e4m3_to_f32((uint8_t)b);
    g_e4_ready = 1;
}

/* one output column over a row of quantized inputs: sum over blocks of ws * (block sum), fp32 or float64 */
static float col_f32(const uint8_t* xq, const uint8_t* wr, const float* ws, int K) {
    float acc = 0.0f;
    for (int b = 0; b < K; b += 128) {
        float p = 0.0f;
        for (int k = b; k < b + 128; ++k) p += g_e4[xq[k]] * g_e4[wr[k]];
        acc += p * ws[b / 128];
    }
    return acc;
}
static double col_f64(const uint8_t* xq, const uint8_t* wr, const float* ws, int K) {
    double acc = 0.0;
    for (int b = 0; b < K; b += 128) {
        double p = 0.0;
        for (int k = b; k < b + 128; ++k) p += (double)g_e4[xq[k]] * (double)g_e4[wr[k]];
        acc += p * (double)ws[b / 128];
    }
    return acc;
}

/*
 * Routed output of one layer. x: [T][K] float (the activations as the kernels read them); pairs (token, local
 * expert, fp32 weight), expert < 0 or >= n skipped. mode 0: fp32 sums (out32), mode 1: float64 (out64).
 * out is accumulated into in pair order per token. Returns 0 or a negative code.
 */
int orc_fp8_moe_forward(const orc_fp8_layer* L, int T, const float* x, int P, const int* pair_token,
                        const int* pair_expert, const float* pair_w, float limit, int mode, float* out32,
                        double* out64, int threads) {
    const int n = L->n, K = L->K, N = L->N;
    if (K % 128 || N % 128 || T < 0 || P < 0 || (mode != 0 && mode != 1)) return -1;
    e4_init();
    uint8_t* qx = (uint8_t*)malloc((size_t)T * K + 1);
    float* sx = (float*)malloc((size_t)T * sizeof(float) + 4);
    float* c32 = mode == 0 ? (float*)calloc((size_t)P * K + 1, sizeof(float)) : NULL;
    double* c64 = mode == 1 ? (double*)calloc((size_t)P * K + 1, sizeof(double)) : NULL;
    if (!qx || !sx || (mode == 0 && !c32) || (mode == 1 && !c64)) return -2;
    orc_quant_rows(x, T, K, qx, sx);
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#endif
#pragma omp parallel
    {
        float* a = (float*)malloc((size_t)N * sizeof(float));
        uint8_t* qa = (uint8_t*)malloc((size_t)N);
#pragma omp for schedule(dynamic, 1)
        for (int j = 0; j < P; ++j) {
            const int e = pair_expert[j], t = pair_token[j];
            if (e < 0 || e >= n || t < 0 || t >= T) continue;
            const uint8_t* xq = qx + (size_t)t * K;
            const uint8_t* w13 = L->w13 + (size_t)e * 2 * N * K;
            const float* s13 = L->w13s + (size_t)e * (2 * N / 128) * (K / 128);
            for (int c = 0; c < N; ++c) {
                const float* sg = s13 + (size_t)(c / 128) * (K / 128);
                const float* su = s13 + (size_t)((N + c) / 128) * (K / 128);
                if (mode == 0) {
                    float g = col_f32(xq, w13 + (size_t)c * K, sg, K) * sx[t];
                    float u = col_f32(xq, w13 + (size_t)(N + c) * K, su, K) * sx[t];
                    if (limit != 0.0f) {
                        g = fminf(g, limit);
                        u = fminf(fmaxf(u, -limit), limit);
                    }
                    const float act = g / (1.0f + (float)exp(-(double)g)) * u;
                    a[c] = orc_h2f(orc_f2h(act));
                } else {
                    double g = col_f64(xq, w13 + (size_t)c * K, sg, K) * (double)sx[t];
                    double u = col_f64(xq, w13 + (size_t)(N + c) * K, su, K) * (double)sx[t];
                    if (limit != 0.0f) {
                        g = fmin(g, (double)limit);
                        u = fmin(fmax(u, -(double)limit), (double)limit);
                    }
                    a[c] = orc_h2f(orc_d2h(g / (1.0 + exp(-g)) * u));
                }
            }
            float sa;
            orc_quant_rows(a, 1, N, qa, &sa);
            const uint8_t* w2 = L->w2 + (size_t)e * K * N;
            const float* s2 = L->w2s + (size_t)e * (K / 128) * (N / 128);
            for (int c = 0; c < K; ++c) {
                const float* sd = s2 + (size_t)(c / 128) * (N / 128);
                if (mode == 0) {
                    const float y = col_f32(qa, w2 + (size_t)c * N, sd, N) * sa;
                    c32[(size_t)j * K + c] = pair_w[j] * y;
                } else {
                    const double y = col_f64(qa, w2 + (size_t)c * N, sd, N) * (double)sa;
                    c64[(size_t)j * K + c] = (double)pair_w[j] * y;
                }
            }
        }
        free(a);
        free(qa);
    }
    for (int j = 0; j < P; ++j) {
        const int e = pair_expert[j], t = pair_token[j];
        if (e < 0 || e >= n || t < 0 || t >= T) continue;
        for (int k = 0; k < K; ++k) {
            if (mode == 0) out32[(size_t)t * K + k] += c32[(size_t)j * K + k];
            else out64[(size_t)t * K + k] += c64[(size_t)j * K + k];
        }
    }
    free(qx);
    free(sx);
    free(c32);
    free(c64);
    return 0;
}
