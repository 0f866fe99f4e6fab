/*
 * CPU oracle for the routed-MoE hot path. TEST INFRASTRUCTURE ONLY: the reference the HIP kernels' results are
 * compared with (tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg). The shipped library never links it.
 *
 * Plain C restatement of the reference's arithmetic:
 *   - EXL3 4-bit trellis format and decode: code/fork/kernels/exl3_format_ref.py:13-27 (closed form), :70-97
 *     (states / unpack); value = fp16(lo) + fp16(hi) with one fp16 rounding (exl3_format_ref.py:54-56).
 *   - 128-point Walsh-Hadamard butterfly, strides 1, 2, ..., 64 in fp32 (code/fork/kernels/exl3.cu:273-284,
 *     code/fork/tests/test_units.py:29-44), r = 0.088388347648f (exl3.cu:37-39).
 *   - input rotation (rot_in / fm_gather): fp16(H(fp16(x * suh)) * r) (exl3.cu:321-349,
 *     code/fork/docs/ref/mia_exl3-fat-kernel/exl3_fat_moe.cu:95-126).
 *   - decode-path epilogues (exl3_moe semantics, SiLU then the limit: code/fork/docs/ref/xl_hadamard_inner.cuh:
 *     280-400, exl3.cu:371-449) and E3 prefill epilogues (limit then SiLU, sigmoid = 1/(1+(float)exp(-(double)g)):
 *     exl3_fat_moe.cu:340-378, 443-457), each evaluated at the rounding points the HIP kernels use.
 *   - float64 layer reference y = ((((x*suh) H) Wq) H) * svh (exl3_format_ref.py:127-131,
 *     code/fork/tests/test_e2e_vs_f64.py:52-75).
 * Threads: OpenMP over experts (one decoded expert per thread at a time).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define MCG_MUL 0xCBAC1FEDu
#define MCG_MASK 0x8FFF8FFFu
#define MCG_FLIP 0x3B603B60u
static const float HAD_R = 0.088388347648f;

/* ---------------------------------------------------------------- fp16 conversions (IEEE binary16, RN-even) */

float orc_h2f(uint16_t h) {
    const uint32_t s = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0x1F) bits = s | 0x7F800000u | (m << 13);                 /* inf / nan */
    else if (e == 0) {
        if (m == 0) bits = s;
        else { float f = (float)m * (1.0f / 16777216.0f); memcpy(&bits, &f, 4); bits |= s; }   /* subnormal */
    } else bits = s | ((e + 112u) << 23) | (m << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* double -> fp16 with one rounding (round to nearest, ties to even) */
uint16_t orc_d2h(double d) {
    uint64_t x;
    memcpy(&x, &d, 8);
    const uint16_t sign = (uint16_t)((x >> 48) & 0x8000u);
    const uint64_t ax = x & 0x7FFFFFFFFFFFFFFFull;
    if (ax >= 0x7FF0000000000000ull) return sign | (ax > 0x7FF0000000000000ull ? 0x7E00 : 0x7C00);
    const double a = fabs(d);
    if (a >= 65520.0) return sign | 0x7C00;                           /* rounds past the largest half */
    if (a < 6.103515625e-05) {                                       /* below 2^-14: subnormal grid 2^-24 */
        const double q = nearbyint(a * 16777216.0);                  /* exact scaling, RN-even */
        return sign | (uint16_t)q;                                   /* q == 1024 is the smallest normal */
    }
    int e;
    const double fr = frexp(a, &e);                                  /* a = fr * 2^e, fr in [0.5, 1) */
    const double q = nearbyint(ldexp(fr, 11));                       /* 11 significant bits, RN-even */
    const double r = ldexp(q, e - 11);
    if (r >= 65520.0) return sign | 0x7C00;
    int e2;
    const double fr2 = frexp(r, &e2);
    const uint32_t mant = (uint32_t)(ldexp(fr2, 11)) & 0x3FFu;
    const uint32_t exp = (uint32_t)(e2 - 1 + 15);
    return sign | (uint16_t)((exp << 10) | mant);
}

uint16_t orc_f2h(float f) { return orc_d2h((double)f); }            /* float is exact in double */

static inline float rh(float f) { return orc_h2f(orc_f2h(f)); }     /* round through fp16 */
static inline float hmul(float a, float b) { return rh(a * b); }     /* fp16 x fp16: the fp32 product is exact */

/* ---------------------------------------------------------------- EXL3 codebook and tile decode */

uint16_t orc_codebook_value(uint32_t s) {
    uint32_t x = (s & 0xFFFFu) * MCG_MUL;
    x = (x & MCG_MASK) ^ MCG_FLIP;
    return orc_d2h((double)orc_h2f((uint16_t)(x & 0xFFFFu)) + (double)orc_h2f((uint16_t)(x >> 16)));
}

void orc_codebook(uint16_t* cb) {
    for (uint32_t s = 0; s < 65536u; ++s) cb[s] = orc_codebook_value(s);
}

/* Position in its 16x16 tile of value p (stream order): ExLlamaV3's fragment order
 * (exl3_format_ref.py:22-23). */
void orc_tile_pos(int p, int* row, int* col) {
    const int l = p >> 3, j = p & 7;
    *row = 2 * (l & 3) + (j & 1) + 8 * ((j >> 1) & 1);
    *col = (l >> 2) + 8 * (j >> 2);
}

/* 16-bit state of value p of a 4-bit tile: the 16 stream bits ending at bit 4p+4 (circular, MSB-first in each
 * little-endian 32-bit word). `words` = the tile's 32 uint32. */
static inline uint32_t tile_state(const uint32_t* words, int p) {
    const int end = 4 * p + 4;                                       /* one past the last bit, stream offset */
    const int start = end - 16;                                      /* may be negative: wraps */
    uint32_t s = 0;
    for (int b = start; b < end; ++b) {
        const int pos = (b + 1024) & 1023;                           /* 1024 bits a tile */
        const uint32_t bit = (words[pos >> 5] >> (31 - (pos & 31))) & 1u;
        s = (s << 1) | bit;
    }
    return s;
}

/* trellis int16 [kt][nt][64] -> W_q fp16 bits [kt*16][nt*16] (row-major, K rows, N columns) */
static uint16_t g_cb[65536];
static float g_cbf[65536];
static float g_cbx[65536];         /* fp16(lo) + fp16(hi) without the final fp16 rounding (exact in fp32) */
static int g_cb_ready = 0;

/* fills the codebook tables once; called before any parallel region */
void orc_init(void) {
    if (g_cb_ready) return;
    orc_codebook(g_cb);
    for (uint32_t s = 0; s < 65536u; ++s) {
        g_cbf[s] = orc_h2f(g_cb[s]);
        uint32_t x = s * MCG_MUL;
        x = (x & MCG_MASK) ^ MCG_FLIP;
        g_cbx[s] = (float)((double)orc_h2f((uint16_t)(x & 0xFFFFu)) + (double)orc_h2f((uint16_t)(x >> 16)));
    }
    g_cb_ready = 1;
}

/* fp16(lo) + fp16(hi) of every state without the final rounding (exact in fp32) */
void orc_codebook_exact(float* cb) {
    orc_init();
    for (uint32_t s = 0; s < 65536u; ++s) cb[s] = g_cbx[s];
}

void orc_unpack(const uint16_t* trellis, int kt, int nt, uint16_t* wq) {
    orc_init();
    const uint16_t* cb = g_cb;
    const int ncol = nt * 16;
#pragma omp parallel for schedule(static)
    for (int a = 0; a < kt; ++a) {
        uint32_t words[32];
        for (int b = 0; b < nt; ++b) {
            const uint16_t* t = trellis + ((size_t)a * nt + b) * 64;
            for (int i = 0; i < 32; ++i) words[i] = (uint32_t)t[2 * i] | ((uint32_t)t[2 * i + 1] << 16);
            for (int p = 0; p < 256; ++p) {
                int r, c;
                orc_tile_pos(p, &r, &c);
                wq[(size_t)(a * 16 + r) * ncol + b * 16 + c] = cb[tile_state(words, p)];
            }
        }
    }
}

static void unpack_f32(const uint16_t* trellis, int kt, int nt, float* w, const float* cbf) {
    const int ncol = nt * 16;
    uint32_t words[32];
    for (int a = 0; a < kt; ++a)
        for (int b = 0; b < nt; ++b) {
            const uint16_t* t = trellis + ((size_t)a * nt + b) * 64;
            for (int i = 0; i < 32; ++i) words[i] = (uint32_t)t[2 * i] | ((uint32_t)t[2 * i + 1] << 16);
            /* word-wise state extraction (the same bits as tile_state, cheaper) */
            for (int l = 0; l < 32; ++l) {
                const uint64_t c = ((uint64_t)words[(l + 31) & 31] << 32) | words[l];
                for (int j = 0; j < 8; ++j) {
                    const uint32_t s = (uint32_t)(c >> (28 - 4 * j)) & 0xFFFFu;
                    int r, cc;
                    orc_tile_pos(8 * l + j, &r, &cc);
                    w[(size_t)(a * 16 + r) * ncol + b * 16 + cc] = cbf[s];
                }
            }
        }
}

/* ---------------------------------------------------------------- Hadamard */

void orc_fwht128(float* v) {
    for (int s = 1; s < 128; s <<= 1)
        for (int i = 0; i < 128; i += 2 * s)
            for (int k = i; k < i + s; ++k) {
                const float a = v[k], b = v[k + s];
                v[k] = a + b;
                v[k + s] = a - b;
            }
}

static void fwht128_d(double* v) {
    for (int s = 1; s < 128; s <<= 1)
        for (int i = 0; i < 128; i += 2 * s)
            for (int k = i; k < i + s; ++k) {
                const double a = v[k], b = v[k + s];
                v[k] = a + b;
                v[k + s] = a - b;
            }
}

/* xr = fp16(H(fp16(x16 * suh16)) * r), one row of n (multiple of 128) */
void orc_rot_in(const uint16_t* x16, const uint16_t* suh16, int n, uint16_t* out16) {
    float blk[128];
    for (int b = 0; b < n; b += 128) {
        for (int i = 0; i < 128; ++i) blk[i] = hmul(orc_h2f(x16[b + i]), orc_h2f(suh16[b + i]));
        orc_fwht128(blk);
        for (int i = 0; i < 128; ++i) out16[b + i] = orc_f2h(blk[i] * HAD_R);
    }
}

/* sigmoid as the HIP kernels define it: 1 / (1 + (float)exp(-(double)g)), IEEE fp32 division */
static inline float sigm(float g) { return 1.0f / (1.0f + (float)exp(-(double)g)); }

/* sigm over the n floats whose bit patterns are first, first + 1, ... (g_out may be NULL); OpenMP threads (0: the
 * runtime's default) */
void orc_sigmoid_bits(uint32_t first, int64_t n, float* g_out, float* s_out, int threads) {
    if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const uint32_t b = first + (uint32_t)i;
        float g;
        memcpy(&g, &b, sizeof g);
        if (g_out) g_out[i] = g;
        s_out[i] = sigm(g);
    }
}

/* ---------------------------------------------------------------- the reference's default (TF_PARITY=1) epilogues
 * code/fork/kernels/exl3.cu:31-32 (TF_PARITY defaults to 1), :351-357 (fp16 SiLU), :371-436 (gate/up epilogue),
 * :455-496 (down epilogue). fp16 arithmetic is IEEE binary16 with one rounding per operation: a product or a sum of
 * two fp16 values is exact in double, so rounding that double once is the correctly rounded fp16 result. The
 * reference's SiLU uses the CUDA half intrinsics h2exp / h2rcp; here exp and the reciprocal are the correctly
 * rounded fp16 values of the exact functions (libm exp and a division in double, each then rounded once to fp16),
 * so an element can differ from the reference by an ulp where an intrinsic is not correctly rounded (the
 * reference's own stage test, code/fork/docs/DESIGN.md:553-554, allows 1 fp16 ulp on 1 % of elements there). */
static inline float h_add(float a, float b) { return orc_h2f(orc_d2h((double)a + (double)b)); }
static inline float h_exp(float a) { return orc_h2f(orc_d2h(exp((double)a))); }
static inline float h_rcp(float a) { return orc_h2f(orc_d2h(1.0 / (double)a)); }
static inline float h_min(float a, float b) { return b < a ? b : a; }
static inline float h_max(float a, float b) { return b > a ? b : a; }

/* x * (1 / (1 + exp(-x))) in fp16, x an fp16 value (exl3.cu:351-357) */
float orc_silu_h(float x) {
    const float e = h_exp(-x);
    const float r = h_rcp(h_add(1.0f, e));
    return hmul(x, r);
}

/* Gate/up epilogue of one pair row with the reference's default rounding points (exl3.cu:371-436): the fp32 GEMV
 * sums zg / zu [N] rounded to fp16, rotated per 128 block in fp32, times r rounded to fp16, times svh in fp16,
 * g = silu_h(g), then (L != 0) u clamped to [fp16(-L), fp16(L)] and g to at most fp16(L), a = g * u * suh_d in
 * fp16, rotated in fp32 and stored as fp16(H(a) * r) into xd [N]. zg / zu are not modified. */
void orc_gateup_epilogue_tf(const float* zg, const float* zu, const uint16_t* svh_g, const uint16_t* svh_u,
                            const uint16_t* suh_d, int N, float limit, uint16_t* xd) {
    float g[128], u[128], v[128];
    const float lo = rh(-limit), hi = rh(limit);
    for (int b0 = 0; b0 < N; b0 += 128) {
        for (int i = 0; i < 128; ++i) { g[i] = rh(zg[b0 + i]); u[i] = rh(zu[b0 + i]); }
        orc_fwht128(g);
        orc_fwht128(u);
        for (int i = 0; i < 128; ++i) {
            float gh = hmul(rh(g[i] * HAD_R), orc_h2f(svh_g[b0 + i]));
            float uh = hmul(rh(u[i] * HAD_R), orc_h2f(svh_u[b0 + i]));
            gh = orc_silu_h(gh);
            if (limit != 0.0f) {
                uh = h_min(h_max(uh, lo), hi);
                gh = h_min(gh, hi);
            }
            v[i] = hmul(hmul(gh, uh), orc_h2f(suh_d[b0 + i]));
        }
        orc_fwht128(v);
        for (int i = 0; i < 128; ++i) xd[b0 + i] = orc_f2h(v[i] * HAD_R);
    }
}

/* Down epilogue of one pair row with the reference's default rounding points (exl3.cu:455-496): the fp32 sums
 * zd [K] rounded to fp16, rotated per 128 block in fp32, times (r * w) and then svh_d in fp32, into out [K]. */
void orc_down_epilogue_tf(const float* zd, const uint16_t* svh_d, uint16_t w16, int K, float* out) {
    float v[128];
    const float rs = HAD_R * orc_h2f(w16);
    for (int b0 = 0; b0 < K; b0 += 128) {
        for (int i = 0; i < 128; ++i) v[i] = rh(zd[b0 + i]);
        orc_fwht128(v);
        for (int i = 0; i < 128; ++i) out[b0 + i] = v[i] * rs * orc_h2f(svh_d[b0 + i]);
    }
}

/* ---------------------------------------------------------------- the kernel-mode epilogues (modes 0, 1, 4) */

/* Gate/up epilogue of one pair row at the HIP kernels' rounding points, from the fp32 GEMV/GEMM sums zg / zu [N]
 * (rotated in place, N a multiple of 128): per 128 block g = (H(zg) * r) * svh_g and u likewise in fp32, then
 *   e3 = 1 (E3, exl3_fat_moe.cu:340-378): g = min(g, L), u = clamp(u, -L, L) iff L != 0, a = sigm(g) * g * u;
 *   e3 = 0 (decode: exl3.cu's fp32 g / u and SiLU, then the limit as exl3_moe, xl_hadamard_inner.cuh:280-400):
 *          s = g * sigm(g), s = min(s, L), u = clamp(u, -L, L) iff L != 0, a = s * u;
 * then fp16(fp16(a) * suh_d) (the fp16 activation and its fp16 product with suh_d, xl_hadamard_inner.cuh:320-400,
 * exl3_fat_moe.cu:370-375), rotated in fp32 and stored as xd = fp16(H(.) * r). */
void orc_gateup_epilogue(float* zg, float* zu, const uint16_t* svh_g, const uint16_t* svh_u, const uint16_t* suh_d,
                         int N, float limit, int e3, uint16_t* xd) {
    float act[128];
    for (int b0 = 0; b0 < N; b0 += 128) {
        orc_fwht128(zg + b0);
        orc_fwht128(zu + b0);
        for (int i = 0; i < 128; ++i) {
            float g = zg[b0 + i] * HAD_R * orc_h2f(svh_g[b0 + i]);
            float u = zu[b0 + i] * HAD_R * orc_h2f(svh_u[b0 + i]);
            float a;
            if (e3) {
                if (limit != 0.0f) {
                    g = fminf(g, limit);
                    u = fminf(fmaxf(u, -limit), limit);
                }
                a = sigm(g) * g * u;
            } else {
                float sl = g * sigm(g);
                if (limit != 0.0f) {
                    sl = fminf(sl, limit);
                    u = fminf(fmaxf(u, -limit), limit);
                }
                a = sl * u;
            }
            act[i] = hmul(rh(a), orc_h2f(suh_d[b0 + i]));
        }
        orc_fwht128(act);
        for (int i = 0; i < 128; ++i) xd[b0 + i] = orc_f2h(act[i] * HAD_R);
    }
}

/* Down epilogue of one pair row (zd [K] rotated in place) into out [K]: e3 = 1 (exl3_fat_moe.cu:443-457):
 * ((H(zd) * r) * svh_d) * w; e3 = 0 (exl3.cu:455-496): H(zd) * (r * w) * svh_d. w = the fp16 router weight. */
void orc_down_epilogue(float* zd, const uint16_t* svh_d, uint16_t w16, int K, int e3, float* out) {
    const float w = orc_h2f(w16);
    const float rs = HAD_R * w;
    for (int b0 = 0; b0 < K; b0 += 128) {
        orc_fwht128(zd + b0);
        for (int i = 0; i < 128; ++i)
            out[b0 + i] = e3 ? zd[b0 + i] * HAD_R * orc_h2f(svh_d[b0 + i]) * w : zd[b0 + i] * rs * orc_h2f(svh_d[b0 + i]);
    }
}

/* ---------------------------------------------------------------- one layer of routed experts */

typedef struct {
    int n, K, N;
    const uint16_t* w13_trellis;   /* [n][2][K/16][N/16][64] */
    const uint16_t* w13_suh;       /* [n][2][K] */
    const uint16_t* w13_svh;       /* [n][2][N] */
    const uint16_t* w2_trellis;    /* [n][N/16][K/16][64] */
    const uint16_t* w2_suh;        /* [n][N] */
    const uint16_t* w2_svh;        /* [n][K] */
} orc_layer;

/*
 * Routed MoE of one layer. pairs: P (token, local expert, fp16 weight) entries, expert < 0 or >= n skipped.
 * mode 0: decode path (exl3_moe semantics: s = silu(g), limit after SiLU: min(s, L), u in [-L, L], iff L != 0;
 *         fp32 epilogues; fp16 at the GEMV inputs xg/xu/xd and at the activation a16).
 * mode 1: E3 prefill path (limit before SiLU: g = min(g, L), u in [-L, L], iff L != 0; sigmoid via double exp).
 * mode 2: float64 reference (test_e2e_vs_f64.py:52-75: double everywhere, exl3_moe's post-SiLU clamp,
 *         weights rounded to fp16 as production passes them).
 * mode 3: float64 reference with the limit before SiLU iff L != 0 (production's python loop, prod:961-1006).
 * mode 4: mode 0 with every weight taken as fp16(lo) + fp16(hi) of its codebook word without the final fp16
 *         rounding (the decode GEMV feeds both halves to the matrix cores, whose fp32 sum is exact).
 * mode 5: the reference's default decode numerics (TF_PARITY=1, exl3.cu:31-32): fp32 GEMV sums over fp16 weights
 *         and inputs, with orc_gateup_epilogue_tf / orc_down_epilogue_tf as the epilogues.
 * out[T][K] (fp32, or double for modes 2/3 through out64) is accumulated into in pair order per token.
 * Returns 0, or -1 on a bad argument.
 */
int orc_moe_forward(const orc_layer* L, int T, const uint16_t* x16, int P, const int* pair_token,
                    const int* pair_expert, const uint16_t* pair_w16, float limit, int mode, float* out32,
                    double* out64, int threads) {
    const int n = L->n, K = L->K, N = L->N;
    if (K % 128 || N % 128 || T < 0 || P < 0) return -1;
    const int KT = K / 16, NT = N / 16;
    const int f64 = mode == 2 || mode == 3;
    if (mode < 0 || mode > 5) return -1;
    orc_init();
    const float* cbt = mode == 4 ? g_cbx : g_cbf;
    /* per-pair contribution rows, summed per token in pair order afterwards (deterministic) */
    float* c32 = f64 ? NULL : (float*)calloc((size_t)P * K, sizeof(float));
    double* c64 = f64 ? (double*)calloc((size_t)P * K, sizeof(double)) : NULL;
    if ((f64 && !c64) || (!f64 && !c32)) return -2;
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#endif
#pragma omp parallel
    {
        float* wg = (float*)malloc((size_t)K * N * sizeof(float));
        float* wu = (float*)malloc((size_t)K * N * sizeof(float));
        float* wd = (float*)malloc((size_t)N * K * sizeof(float));
        float* xs = (float*)malloc((size_t)K * 2 * sizeof(float));
        double* xd64 = (double*)malloc((size_t)(2 * K + 4 * N) * sizeof(double));
        float* tmp = (float*)malloc((size_t)(4 * N + 2 * K) * sizeof(float));
        uint16_t* h16 = (uint16_t*)malloc((size_t)(2 * K + N) * sizeof(uint16_t));
#pragma omp for schedule(dynamic, 1)
        for (int e = 0; e < n; ++e) {
            int any = 0;
            for (int j = 0; j < P; ++j) any |= pair_expert[j] == e;
            if (!any) continue;
            unpack_f32(L->w13_trellis + ((size_t)e * 2 + 0) * KT * NT * 64, KT, NT, wg, cbt);
            unpack_f32(L->w13_trellis + ((size_t)e * 2 + 1) * KT * NT * 64, KT, NT, wu, cbt);
            unpack_f32(L->w2_trellis + (size_t)e * NT * KT * 64, NT, KT, wd, cbt);
            const uint16_t* suh_g = L->w13_suh + ((size_t)e * 2 + 0) * K;
            const uint16_t* suh_u = L->w13_suh + ((size_t)e * 2 + 1) * K;
            const uint16_t* svh_g = L->w13_svh + ((size_t)e * 2 + 0) * N;
            const uint16_t* svh_u = L->w13_svh + ((size_t)e * 2 + 1) * N;
            const uint16_t* suh_d = L->w2_suh + (size_t)e * N;
            const uint16_t* svh_d = L->w2_svh + (size_t)e * K;
            for (int j = 0; j < P; ++j) {
                if (pair_expert[j] != e) continue;
                const int t = pair_token[j];
                if (t < 0 || t >= T) continue;
                const uint16_t* xr = x16 + (size_t)t * K;
                if (!f64) {
                    float* zg = tmp;
                    float* zu = tmp + N;
                    float* zd = tmp + 4 * N;
                    uint16_t* xg = h16;
                    uint16_t* xu = h16 + K;
                    uint16_t* xdd = h16 + 2 * K;
                    orc_rot_in(xr, suh_g, K, xg);
                    orc_rot_in(xr, (mode == 1) ? suh_g : suh_u, K, xu);   /* E3 gathers once with gate's suh */
                    for (int c = 0; c < N; ++c) { zg[c] = 0.f; zu[c] = 0.f; }
                    for (int k = 0; k < K; ++k) {
                        const float a = orc_h2f(xg[k]), b = orc_h2f(xu[k]);
                        const float* rg = wg + (size_t)k * N;
                        const float* ru = wu + (size_t)k * N;
                        for (int c = 0; c < N; ++c) { zg[c] += a * rg[c]; zu[c] += b * ru[c]; }
                    }
                    if (mode == 5) orc_gateup_epilogue_tf(zg, zu, svh_g, svh_u, suh_d, N, limit, xdd);
                    else orc_gateup_epilogue(zg, zu, svh_g, svh_u, suh_d, N, limit, mode == 1, xdd);
                    for (int c = 0; c < K; ++c) zd[c] = 0.f;
                    for (int k = 0; k < N; ++k) {
                        const float a = orc_h2f(xdd[k]);
                        const float* rd = wd + (size_t)k * K;
                        for (int c = 0; c < K; ++c) zd[c] += a * rd[c];
                    }
                    float* dst = c32 + (size_t)j * K;
                    if (mode == 5) orc_down_epilogue_tf(zd, svh_d, pair_w16[j], K, dst);
                    else orc_down_epilogue(zd, svh_d, pair_w16[j], K, mode == 1, dst);
                } else {
                    /* float64: y = ((((x*suh) H) Wq) H) * svh per projection */
                    const double rr = 1.0 / sqrt(128.0);
                    double* hg = xd64;
                    double* hu = xd64 + K;
                    double* g = xd64 + 2 * K;
                    double* u = g + N;
                    double* a = u + N;
                    for (int k = 0; k < K; ++k) {
                        hg[k] = (double)orc_h2f(xr[k]) * (double)orc_h2f(suh_g[k]);
                        hu[k] = (double)orc_h2f(xr[k]) * (double)orc_h2f(suh_u[k]);
                    }
                    for (int b0 = 0; b0 < K; b0 += 128) { fwht128_d(hg + b0); fwht128_d(hu + b0); }
                    for (int k = 0; k < K; ++k) { hg[k] *= rr; hu[k] *= rr; }
                    for (int c = 0; c < N; ++c) { g[c] = 0.0; u[c] = 0.0; }
                    for (int k = 0; k < K; ++k) {
                        const float* rg = wg + (size_t)k * N;
                        const float* ru = wu + (size_t)k * N;
                        for (int c = 0; c < N; ++c) { g[c] += hg[k] * rg[c]; u[c] += hu[k] * ru[c]; }
                    }
                    for (int b0 = 0; b0 < N; b0 += 128) { fwht128_d(g + b0); fwht128_d(u + b0); }
                    for (int c = 0; c < N; ++c) {
                        double gv = g[c] * rr * (double)orc_h2f(svh_g[c]);
                        double uv = u[c] * rr * (double)orc_h2f(svh_u[c]);
                        double s;
                        if (mode == 3) {
                            if (limit != 0.0f) {
                                gv = fmin(gv, (double)limit);
                                uv = fmin(fmax(uv, -(double)limit), (double)limit);
                            }
                            s = gv / (1.0 + exp(-gv));
                        } else {
                            s = gv / (1.0 + exp(-gv));
                            if (limit != 0.0f) {
                                s = fmin(s, (double)limit);
                                uv = fmin(fmax(uv, -(double)limit), (double)limit);
                            }
                        }
                        a[c] = s * uv * (double)orc_h2f(suh_d[c]);
                    }
                    for (int b0 = 0; b0 < N; b0 += 128) fwht128_d(a + b0);
                    double* dd = (double*)malloc((size_t)K * sizeof(double));
                    for (int c = 0; c < K; ++c) dd[c] = 0.0;
                    for (int k = 0; k < N; ++k) {
                        const double av = a[k] * rr;
                        const float* rd = wd + (size_t)k * K;
                        for (int c = 0; c < K; ++c) dd[c] += av * rd[c];
                    }
                    for (int b0 = 0; b0 < K; b0 += 128) fwht128_d(dd + b0);
                    const double w = (double)orc_h2f(pair_w16[j]);
                    double* dst = c64 + (size_t)j * K;
                    for (int c = 0; c < K; ++c) dst[c] = dd[c] * rr * (double)orc_h2f(svh_d[c]) * w;
                    free(dd);
                }
            }
        }
        free(wg); free(wu); free(wd); free(xs); free(xd64); free(tmp); free(h16);
    }
    for (int j = 0; j < P; ++j) {
        const int e = pair_expert[j], t = pair_token[j];
        if (e < 0 || e >= n || t < 0 || t >= T) continue;
        if (f64) {
            double* o = out64 + (size_t)t * K;
            const double* c = c64 + (size_t)j * K;
            for (int k = 0; k < K; ++k) o[k] += c[k];
        } else {
            float* o = out32 + (size_t)t * K;
            const float* c = c32 + (size_t)j * K;
            for (int k = 0; k < K; ++k) o[k] += c[k];
        }
    }
    free(c32);
    free(c64);
    return 0;
}

/* exp as the HIP kernels round it: (float)exp((double)a) */
float orc_expf_via_double(float a) { return (float)exp((double)a); }
