// Router and token->expert permutation kernels.
//
// router_logits  logits[t][e] = bf16(x[t] . W[e]) widened to fp32: the bf16 products summed in float64 (exact for
//                router-sized operands, so independent of the order) and rounded to bf16 through fp32.
//                Replaces F.linear(x, W).to(float32) (code/fork/docs/BF16_GEMV.md:27,38).
// router_topk    vLLM grouped_topk with n_group = topk_group = 1 as restated by code/fork/docs/ref/tf_glue.py:371-401:
//                score = sigmoid(logit), pick the topk largest score + bias (lower id first among equals),
//                w = score / (sum of picked scores + 1e-20) * scale, one wave per token.
// route_*        map_topk_to_local (code/fork/docs/prod_exl3_reference.py:936-958), counts, exclusive scan, and the
//                stable sorted position of every pair (pairs grouped by local id, the sentinel group last, inside a
//                group by pair index; code/fork/kernels/exl3.cu:742-775), plus the row-segment table
//                (code/fork/kernels/exl3.cu:529-566) with a caller-chosen segment height.
#include <algorithm>

#include "common.cuh"
#include "mi355moe_internal.h"

namespace mi355moe {

// ------------------------------------------------------------------------------------------------ router GEMV

constexpr int RL_TCHUNK = 8;   // tokens per pass
constexpr int RL_MAXC = 16;    // K chunks of 512 (K <= 8192)

// The value of lane l ^ M for a double (its two words moved by xor_lane).
template <int M>
__device__ __forceinline__ double xor_lane_f64(double v, int lane) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = __builtin_bit_cast(uint32_t, xor_lane<M>(__builtin_bit_cast(float, (uint32_t)u), lane));
    const uint32_t hi = __builtin_bit_cast(uint32_t, xor_lane<M>(__builtin_bit_cast(float, (uint32_t)(u >> 32)), lane));
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// Sums over the 64 lanes of V values per lane (V a power of two <= 64), by halving exchanges: at distance M a lane
// keeps half of its W live values (the upper half where lane & M), adds its partner's copy of that half and sends the
// other; after log2(V) such steps (M = 32, 16, ...) each lane holds one value v = lane / (64 / V) in acc[0], and
// butterflies over the remaining distances finish its sum in every lane of its group (V - 1 exchanges in all instead
// of 6 V).
template <int V, int W = V, int M = 32>
__device__ __forceinline__ void wave_sum_scatter(double (&acc)[V], int lane) {
    static_assert(V >= 1 && V <= 64 && (V & (V - 1)) == 0 && W >= 1 && W <= V, "a power of two <= 64");
    if constexpr (M >= 1) {
        if constexpr (W >= 2) {
            const bool up = (lane & M) != 0;
#pragma unroll
            for (int i = 0; i < W / 2; ++i) {
                const double lo = acc[i], hi = acc[W / 2 + i];
                acc[i] = (up ? hi : lo) + xor_lane_f64<M>(up ? lo : hi, lane);
            }
            wave_sum_scatter<V, W / 2, M / 2>(acc, lane);
        } else {
            acc[0] = acc[0] + xor_lane_f64<M>(acc[0], lane);
            wave_sum_scatter<V, 1, M / 2>(acc, lane);
        }
    }
}

// The router logit as production returns it: F.linear in bf16 rounds the dot product to bf16, .to(float32) widens
// it back (code/fork/docs/BF16_GEMV.md:27,38; the reference's router oracle is (X.double() @ W.t()).to(bfloat16),
// code/fork/tests/router_topk_agreement.py:82, and torch narrows a double to bf16 through fp32). `dot` is the
// float64 sum of the bf16 products; (float) rounds it to nearest even, f32_to_bf16 likewise.
__device__ __forceinline__ float router_round(double dot) { return bf16_to_f32(f32_to_bf16((float)dot)); }

// One workgroup per expert, one wave per 512-wide chunk c of K. Every bf16 x bf16 product is exact in fp32 and its
// significand has at most 16 bits. A float64 partial sum of up to K <= 8192 such terms therefore needs no rounding
// while the terms' exponents span at most 53 - 16 - 13 = 24 binades (a sufficient condition, not a necessary one):
// then the float64 sum is the exact dot product whatever the order, and the bf16 logit is that of the exact value.
// Router-sized operands (x ~ N(0, 1), weights ~ N(0, 0.02)) rarely exceed it, but outlier-heavy hidden states can;
// beyond it the sums of this kernel and of router_gemm_f64_kernel (another order) may differ in their last float64
// bits, which changes the bf16 logit only when the exact value lies within those bits of a rounding boundary of the
// fp32 and bf16 roundings that follow (vanishingly rare, not excluded). Lane l of chunk c accumulates
// k = 512c + 8l + i, i = 0..7; the 64 lane partials are combined by the xor butterfly m = 32, 16, ..., 1; the chunk
// sums are then added in chunk order c = 0, 1, ... (wave 0 adds them from LDS). Waves past K/512 only join the
// barriers. The logits of experts e0 .. e0 + NE - 1 (those below E) for every token. COH: stored as device-coherent
// words (read back by another workgroup of the same grid). SCORE: the stored value is the score sigmoid(logit),
// computed as the top-k does ((float)(1 / (1 + exp(-(double)logit)))), instead of the logit.
template <bool COH = false, int NE = 1, bool SCORE = false>
__device__ __forceinline__ void logits_body(const uint16_t* __restrict__ x, int64_t x_stride,
                                            const uint16_t* __restrict__ w, int T, int K, int E, int e0,
                                            float* __restrict__ logits) {
    __shared__ double part[RL_MAXC][NE * RL_TCHUNK];
    const int lane = threadIdx.x & 63;
    const int c = threadIdx.x >> 6;                 // chunk of this wave
    const int chunks = K / 512;
    const int k0 = c * 512 + lane * 8;
    for (int t0 = 0; t0 < T; t0 += RL_TCHUNK) {
        if (c < chunks) {
            // the pass's token rows and the weight chunks are all loaded before any is used (one memory latency
            // per pass; later passes find the weights in L2)
            u32x4 xv[RL_TCHUNK];
#pragma unroll
            for (int tt = 0; tt < RL_TCHUNK; ++tt)
                xv[tt] = t0 + tt < T ? *reinterpret_cast<const u32x4*>(x + (size_t)(t0 + tt) * x_stride + k0)
                                     : u32x4{0u, 0u, 0u, 0u};
            double wd[NE][8];
#pragma unroll
            for (int q = 0; q < NE; ++q) {
                const u32x4 wv = *reinterpret_cast<const u32x4*>(w + (size_t)min(e0 + q, E - 1) * K + k0);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    wd[q][2 * i] = (double)__builtin_bit_cast(float, wv[i] << 16);
                    wd[q][2 * i + 1] = (double)__builtin_bit_cast(float, wv[i] & 0xFFFF0000u);
                }
            }
            double acc[NE * RL_TCHUNK];                               // value v = q RL_TCHUNK + tt
#pragma unroll
            for (int tt = 0; tt < RL_TCHUNK; ++tt) {
                double xd[8];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    xd[2 * i] = (double)__builtin_bit_cast(float, xv[tt][i] << 16);
                    xd[2 * i + 1] = (double)__builtin_bit_cast(float, xv[tt][i] & 0xFFFF0000u);
                }
#pragma unroll
                for (int q = 0; q < NE; ++q) {
                    double a = 0.0;
#pragma unroll
                    for (int i = 0; i < 8; ++i) a = __builtin_fma(xd[i], wd[q][i], a);
                    acc[q * RL_TCHUNK + tt] = a;
                }
            }
            // sums over the 64 lanes: value v ends in lane 4 v (for 16 values; see wave_sum_scatter)
            constexpr int V = NE * RL_TCHUNK;
            wave_sum_scatter<V>(acc, lane);
            constexpr int SPREAD = 64 / V;
            if ((lane & (SPREAD - 1)) == 0) part[c][lane / SPREAD] = acc[0];
        }
        __syncthreads();
        const int q = (int)threadIdx.x / RL_TCHUNK, tt = (int)threadIdx.x % RL_TCHUNK;
        if (q < NE && e0 + q < E && t0 + tt < T) {
            double dot = part[0][threadIdx.x];
            for (int cc = 1; cc < chunks; ++cc) dot = dot + part[cc][threadIdx.x];
            float sum = router_round(dot);
            if (SCORE) sum = (float)(1.0 / (1.0 + exp(-(double)sum)));
            float* dst = logits + (size_t)(t0 + tt) * E + e0 + q;
            if (COH) st_coherent(dst, sum);
            else *dst = sum;
        }
        __syncthreads();
    }
}

// Large-T router GEMM on the float64 matrix cores (v_mfma_f64_16x16x4_f64): a wave computes 16 tokens x 32 experts
// (two 16 x 16 blocks) over all of K. The bf16 inputs are widened exactly to float64 and every product and sum of the
// MFMA is float64, so -- while the terms span at most 24 binades, as in logits_body -- the sums are the exact dot
// products whatever their order, and the logits equal the GEMV kernel's bit for bit. The reduction order is
// free, so lane group g = lane / 16 (the MFMA's k index) walks its own contiguous quarter of K, k = g K / 4 + j,
// with 16-byte loads of 8 consecutive bf16. MFMA layouts (16 x 16 x 4, float64): A[i][k] from lane i + 16 k, B[k][j]
// from lane j + 16 k, D[i][j] in lane j + 16 (i % 4), element i / 4 (rows interleaved by 4, unlike the 16 x 16
// layouts of the narrower types).
typedef double f64x4 __attribute__((ext_vector_type(4)));
constexpr int RG_TOK = 16, RG_EXP = 32;   // tokens x experts per wave
__global__ __launch_bounds__(256) void router_gemm_f64_kernel(const uint16_t* __restrict__ x, int64_t x_stride,
                                                              const uint16_t* __restrict__ w, int T, int K, int E,
                                                              float* __restrict__ logits) {
    const int lane = threadIdx.x & 63;
    const int tiles_e = (E + RG_EXP - 1) / RG_EXP;
    const int tile = (int)blockIdx.x * 4 + (int)(threadIdx.x >> 6);
    const int t0 = (tile / tiles_e) * RG_TOK, e0 = (tile % tiles_e) * RG_EXP;
    if (t0 >= T) return;                                             // uniform over the wave (no block barrier)
    const int g = lane >> 4, r = lane & 15;
    const int kq = K >> 2;
    const uint16_t* xa = x + (size_t)min(t0 + r, T - 1) * x_stride + (size_t)g * kq;
    const uint16_t* wb0 = w + (size_t)min(e0 + r, E - 1) * K + (size_t)g * kq;
    const uint16_t* wb1 = w + (size_t)min(e0 + 16 + r, E - 1) * K + (size_t)g * kq;
    f64x4 acc0 = {0.0, 0.0, 0.0, 0.0}, acc1 = {0.0, 0.0, 0.0, 0.0};
    for (int k = 0; k < kq; k += 8) {
        const u32x4 av = *reinterpret_cast<const u32x4*>(xa + k);
        const u32x4 b0 = *reinterpret_cast<const u32x4*>(wb0 + k);
        const u32x4 b1 = *reinterpret_cast<const u32x4*>(wb1 + k);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int sh = (q & 1) ? 0 : 16;                         // element q of a dword pair: low half first
            const uint32_t m = 0xFFFF0000u;
            const double a = (double)__builtin_bit_cast(float, (av[q >> 1] << sh) & m);
            const double c0 = (double)__builtin_bit_cast(float, (b0[q >> 1] << sh) & m);
            const double c1 = (double)__builtin_bit_cast(float, (b1[q >> 1] << sh) & m);
            acc0 = __builtin_amdgcn_mfma_f64_16x16x4f64(a, c0, acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f64_16x16x4f64(a, c1, acc1, 0, 0, 0);
        }
    }
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        const int t = t0 + g + 4 * v;
        if (t >= T) continue;
        if (e0 + r < E) logits[(size_t)t * E + e0 + r] = router_round(acc0[v]);
        if (e0 + 16 + r < E) logits[(size_t)t * E + e0 + 16 + r] = router_round(acc1[v]);
    }
}
constexpr int RG_MIN_T = 256;   // from this many tokens the MFMA GEMM beats the GEMV kernel

__global__ __launch_bounds__(1024) void router_logits_kernel(const uint16_t* __restrict__ x, int64_t x_stride,
                                                             const uint16_t* __restrict__ w, int T, int K, int E,
                                                             float* __restrict__ logits) {
    logits_body(x, x_stride, w, T, K, E, blockIdx.x, logits);
}

// ------------------------------------------------------------------------------------------------ router top-k

constexpr int TOPK_MAX_E = 1024;   // experts per token row
constexpr int TOPK_MAX_K = 32;

// ------------------------------------------------------------------------------------------------ permutation

template <typename IT>
__device__ __forceinline__ int local_id(IT raw, const int64_t* __restrict__ emap, int64_t n_global, int n) {
    const int64_t id = (int64_t)raw;
    if (!emap) return (id < 0 || id >= n) ? n : (int)id;
    const int64_t hi = n_global > 0 ? n_global - 1 : 0;
    const int64_t safe = id < 0 ? 0 : (id > hi ? hi : id);
    const int64_t mapped = n_global ? emap[safe] : (int64_t)n;
    return (id < 0 || id >= n_global || mapped < 0 || mapped >= n) ? n : (int)mapped;
}

__device__ __forceinline__ uint16_t weight_f16(const void* w, int wdt, int j) {
    float f;
    if (wdt == DT_F32) f = reinterpret_cast<const float*>(w)[j];
    else if (wdt == DT_BF16) f = bf16_to_f32(reinterpret_cast<const uint16_t*>(w)[j]);
    else return reinterpret_cast<const uint16_t*>(w)[j];
    return (uint16_t)h_as_u16((_Float16)f);
}

__device__ __forceinline__ float weight_f32(const void* w, int wdt, int j) {
    if (wdt == DT_F32) return reinterpret_cast<const float*>(w)[j];
    if (wdt == DT_BF16) return bf16_to_f32(reinterpret_cast<const uint16_t*>(w)[j]);
    return (float)u16_as_h(reinterpret_cast<const uint16_t*>(w)[j]);
}

// block-wide inclusive scan of one int per thread (blockDim.x a multiple of 64, <= 1024)
// Inclusive scan over the 64 lanes of a wave by DPP (no LDS): shifts by 1, 2, 4, 8 inside each 16-lane row (lanes
// without a source add 0), then lane 15 of rows 0 and 2 into rows 1 and 3 and lane 31 into rows 2 and 3.
__device__ __forceinline__ int wave_scan_incl(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);   // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);   // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);   // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true);   // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31
    return v;
}

__device__ __forceinline__ int block_scan_incl(int v, int* tot, int& total) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
    v = wave_scan_incl(v);
    if (lane == 63) tot[wv] = v;
    __syncthreads();
    if (wv == 0) {
        int s = wave_scan_incl(lane < nw ? tot[lane] : 0);
        if (lane < nw) tot[lane] = s;
    }
    __syncthreads();
    const int pre = wv ? tot[wv - 1] : 0;
    total = tot[nw - 1];
    __syncthreads();
    return v + pre;
}

// Segment table from per-expert counts held in `cnt` (shared, [n]) and their starts: every expert with
// max(0, Rmin) < c <= R gets ceil(c / seg) segments (expert, first row, rows). Called by every thread of the block.
__device__ void build_segments(const int* cnt, const int* start, int n, int R, int seg, int S_cap,
                               int* __restrict__ seg_expert, int* __restrict__ seg_row0, int* __restrict__ seg_rows,
                               int* __restrict__ nseg_out, int* tot, int Rmin = 0) {
    int run = 0;
    for (int base = 0; base < n; base += blockDim.x) {
        const int e = base + threadIdx.x;
        const int c = e < n ? cnt[e] : 0;
        const bool elig = e < n && c > Rmin && c > 0 && c <= R;
        const int ns = elig ? (c + seg - 1) / seg : 0;
        int stot;
        const int sinc = block_scan_incl(ns, tot, stot);
        const int soff = run + sinc - ns;
        if (elig)
            for (int q = 0; q < ns; ++q) {
                const int s = soff + q;
                if (s < S_cap) {
                    seg_expert[s] = e;
                    seg_row0[s] = start[e] + seg * q;
                    seg_rows[s] = min(seg, c - seg * q);
                }
            }
        run += stot;
    }
    if (threadIdx.x == 0) nseg_out[0] = run < S_cap ? run : S_cap;
}

// Zeroes this call's split-K arrival counters (a grid-stride fill by the first kernel of the call).
__device__ __forceinline__ void zero_counters(const RouteArgs& a) {
    if (!a.zero) return;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.zero_words;
         i += (int64_t)gridDim.x * blockDim.x)
        a.zero[i] = 0u;
}

// One block does the whole permutation (P <= ROUTE_SMALL_MAX_P). Shared memory sh: local[P], cnt[n+1], start[n+1].
template <typename IT>
__device__ void route_small_body(const RouteArgs& a, int* sh) {
    __shared__ int tot[16];
    int* loc = sh;
    int* cnt = sh + a.P;
    int* start = cnt + (a.n + 1);
    const IT* ids = reinterpret_cast<const IT*>(a.ids);
    if (a.zero)
        for (int64_t i = threadIdx.x; i < a.zero_words; i += blockDim.x) a.zero[i] = 0u;
    for (int e = threadIdx.x; e <= a.n; e += blockDim.x) cnt[e] = 0;
    __syncthreads();
    for (int j = threadIdx.x; j < a.P; j += blockDim.x) {
        const int l = local_id<IT>(ids[j], a.emap, a.n_global, a.n);
        loc[j] = l;
        atomicAdd(&cnt[l], 1);
    }
    __syncthreads();
    int run = 0;
    for (int base = 0; base <= a.n; base += blockDim.x) {
        const int e = base + threadIdx.x;
        const int c = e <= a.n ? cnt[e] : 0;
        int ctot;
        const int cinc = block_scan_incl(c, tot, ctot);
        if (e <= a.n) start[e] = run + cinc - c;
        run += ctot;
    }
    __syncthreads();
    if (a.counts)
        for (int e = threadIdx.x; e <= a.n; e += blockDim.x) a.counts[e] = cnt[e];
    build_segments(cnt, start, a.n, a.R, a.seg, a.S_cap, a.seg_expert, a.seg_row0, a.seg_rows, a.nseg, tot, a.Rmin);
    for (int j = threadIdx.x; j < a.P; j += blockDim.x) {
        const int l = loc[j];
        int rank = 0;                                                // earlier pairs with the same local id
        const int4* l4 = reinterpret_cast<const int4*>(loc);
#pragma unroll 8
        for (int i4 = 0; i4 < (j >> 2); ++i4) {
            const int4 v = l4[i4];
            rank += (v.x == l) + (v.y == l) + (v.z == l) + (v.w == l);
        }
        for (int i = j & ~3; i < j; ++i) rank += loc[i] == l;
        const int pos = start[l] + rank;
        a.tok[pos] = j / a.topk;
        a.w16[pos] = weight_f16(a.w, a.wdt, j);
        if (a.w32) a.w32[pos] = weight_f32(a.w, a.wdt, j);
        a.pe[pos] = (l < a.n && cnt[l] <= a.R && cnt[l] > a.Rmin) ? l : -1;
        a.inv[j] = pos;
    }
}

// One compare-exchange stage of an ascending bitonic sort across the wave: partner = lane ^ S; k = the size of the
// sequences being merged.
template <int S>
__device__ __forceinline__ uint32_t bitonic_stage(uint32_t key, int lane, int k) {
    const uint32_t o = __builtin_bit_cast(uint32_t, xor_lane<S>(__builtin_bit_cast(float, key), lane));
    const bool up = (lane & k) == 0, low = (lane & S) == 0;
    return (low == up) ? (o < key ? o : key) : (o > key ? o : key);
}

// route_small_body for the picks of a top-k (P <= 64 pairs, every token's picks distinct experts, seg >= T rows):
// the workgroup zeroes the call's counters and the counts, then wave 0 alone sorts the pairs' keys (local id << 6 |
// pair index) with a bitonic network across its lanes, which is the stable sorted order of route_small_body; an
// expert then has c <= T <= seg pairs, so each eligible expert (c <= R, not the sentinel) is one segment, found as a
// run of equal ids. The tables equal route_small_body's.
template <typename IT>
__device__ void route_wave64(const RouteArgs& a) {
    if (a.zero)
        for (int64_t i = threadIdx.x; i < a.zero_words; i += blockDim.x) a.zero[i] = 0u;
    if (a.counts)
        for (int e = threadIdx.x; e <= a.n; e += blockDim.x) a.counts[e] = 0;
    __syncthreads();
    if (threadIdx.x >= 64) return;
    const int lane = threadIdx.x;
    const IT* ids = reinterpret_cast<const IT*>(a.ids);
    uint32_t key = 0xFFFFFFFFu;
    if (lane < a.P) key = ((uint32_t)local_id<IT>(ids[lane], a.emap, a.n_global, a.n) << 6) | (uint32_t)lane;
    key = bitonic_stage<1>(key, lane, 2);
    key = bitonic_stage<2>(key, lane, 4);
    key = bitonic_stage<1>(key, lane, 4);
    key = bitonic_stage<4>(key, lane, 8);
    key = bitonic_stage<2>(key, lane, 8);
    key = bitonic_stage<1>(key, lane, 8);
    key = bitonic_stage<8>(key, lane, 16);
    key = bitonic_stage<4>(key, lane, 16);
    key = bitonic_stage<2>(key, lane, 16);
    key = bitonic_stage<1>(key, lane, 16);
    key = bitonic_stage<16>(key, lane, 32);
    key = bitonic_stage<8>(key, lane, 32);
    key = bitonic_stage<4>(key, lane, 32);
    key = bitonic_stage<2>(key, lane, 32);
    key = bitonic_stage<1>(key, lane, 32);
    key = bitonic_stage<32>(key, lane, 64);
    key = bitonic_stage<16>(key, lane, 64);
    key = bitonic_stage<8>(key, lane, 64);
    key = bitonic_stage<4>(key, lane, 64);
    key = bitonic_stage<2>(key, lane, 64);
    key = bitonic_stage<1>(key, lane, 64);
    const bool valid = lane < a.P;                                   // sorted position lane holds a pair
    const int l = (int)(key >> 6), j = (int)(key & 63u);
    const int lprev = __shfl(l, lane > 0 ? lane - 1 : 0, 64);
    const bool start = valid && (lane == 0 || lprev != l);
    const uint64_t smask = __ballot(start);
    const uint64_t above = lane == 63 ? 0ull : smask >> (lane + 1);
    const int c = (above ? lane + 1 + __builtin_ctzll(above) : a.P) - lane;   // run length, at run starts
    const bool elig = start && l < a.n && c <= a.R && c > a.Rmin;
    const uint64_t emask = __ballot(elig);
    const uint64_t upto = smask & (lane == 63 ? ~0ull : ((1ull << (lane + 1)) - 1));
    const int rs = upto ? 63 - __builtin_clzll(upto) : 0;           // this lane's run start
    const bool run_elig = __shfl(elig ? 1 : 0, rs, 64) != 0;
    if (valid) {
        a.tok[lane] = j / a.topk;
        a.w16[lane] = weight_f16(a.w, a.wdt, j);
        if (a.w32) a.w32[lane] = weight_f32(a.w, a.wdt, j);
        a.pe[lane] = run_elig ? l : -1;
        a.inv[j] = lane;
    }
    if (elig) {
        const int sg = __builtin_popcountll(emask & ((1ull << lane) - 1));
        if (sg < a.S_cap) {
            a.seg_expert[sg] = l;
            a.seg_row0[sg] = lane;
            a.seg_rows[sg] = c;
        }
    }
    if (start && a.counts) a.counts[l] = c;
    if (lane == 0) {
        const int ns = __builtin_popcountll(emask);
        a.nseg[0] = ns < a.S_cap ? ns : a.S_cap;
    }
}

template <typename IT>
__global__ __launch_bounds__(1024) void route_small_kernel(RouteArgs a) {
    extern __shared__ int sh[];
    route_small_body<IT>(a, sh);
}

// ------------------------------------------------------------------------------------------------ top-k + permutation

// Order key of a candidate: the choice key (score + bias; -0 made +0) mapped to an unsigned integer with the same
// order. Every finite key maps above 0, so 0 marks an empty or taken slot. Among equal keys the lower expert id is
// picked first (the reference's order).
__device__ __forceinline__ uint32_t topk_key(float key) {
    const uint32_t b = __builtin_bit_cast(uint32_t, key + 0.0f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Maximum / minimum of a 32-bit value over the wave, returned in every lane: rotations by 1, 2, 4, 8 inside each
// 16-lane row (DPP, no LDS), then the four row results by readlane.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x121, 0xF, 0xF, true));   // row_ror:1
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x122, 0xF, 0xF, true));   // row_ror:2
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x124, 0xF, 0xF, true));   // row_ror:4
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, true));   // row_ror:8
    const uint32_t a = max((uint32_t)__builtin_amdgcn_readlane((int)v, 0), (uint32_t)__builtin_amdgcn_readlane((int)v, 16));
    const uint32_t b = max((uint32_t)__builtin_amdgcn_readlane((int)v, 32), (uint32_t)__builtin_amdgcn_readlane((int)v, 48));
    return max(a, b);
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
    v = min(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x121, 0xF, 0xF, true));
    v = min(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x122, 0xF, 0xF, true));
    v = min(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x124, 0xF, 0xF, true));
    v = min(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, true));
    const uint32_t a = min((uint32_t)__builtin_amdgcn_readlane((int)v, 0), (uint32_t)__builtin_amdgcn_readlane((int)v, 16));
    const uint32_t b = min((uint32_t)__builtin_amdgcn_readlane((int)v, 32), (uint32_t)__builtin_amdgcn_readlane((int)v, 48));
    return min(a, b);
}

// One wave's top-k of one token (E <= 1024 candidates, lane l holding candidates l + 64 j). Every load of the row (and
// of the bias) is issued before the first is used, so the row costs one memory latency. Each lane sorts its keys once
// (descending, the lower j first among equal keys, hence the lower id). Then topk rounds: the wave maximum of the
// lanes' best keys and the winner among the lanes holding it -- the only one, or with equal keys in several lanes
// the lowest id, by a wave minimum. The winner's lane drops it, so picks come largest first, lower id on ties (the
// reference's order). Scores s = sigmoid(logit)
// (through double exp) go to sco [E] for the weights; weights are the picks' scores renormalised over their total
// (summed sequentially in pick order, + 1e-20, correctly rounded division) and scaled.
// J >= ceil(E / 64); COH: coherent loads of the row; SCORE: the row holds the scores sigmoid(logit) already
template <int J, bool COH = false, bool SCORE = false>
__device__ __forceinline__ void topk_wave(const float* __restrict__ lrow, int E, const float* __restrict__ bias,
                                          int topk, float scale, int renorm, float* sco, int32_t* __restrict__ ids_row,
                                          float* __restrict__ wts_row, int* ids_sh, float* wts_sh) {
    const int lane = threadIdx.x & 63;
    float lv[J], bv[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {                                     // clamped addresses: every load in bounds
        const int e = min(lane + 64 * j, E - 1);
        lv[j] = COH ? ld_coherent(lrow + e) : lrow[e];
        bv[j] = bias ? bias[e] : 0.f;
    }
    uint32_t key[J];
    int jo[J];                                                        // key i's candidate index j
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int e = lane + 64 * j;
        key[j] = 0u;
        jo[j] = j;
        if (e < E) {
            const float sv = SCORE ? lv[j] : (float)(1.0 / (1.0 + exp(-(double)lv[j])));
            sco[e] = sv;
            key[j] = topk_key(sv + bv[j]);
        }
    }
    int mine_e = 0;                                                   // lane k: the k-th pick
    if constexpr (J <= 8) {
        // each lane's keys in descending order, equal keys in ascending j (odd-even transposition: J rounds of
        // adjacent swaps of strictly smaller keys, which keeps equal keys in their order); its best is key[0]
#pragma unroll
        for (int r = 0; r < J; ++r)
#pragma unroll
            for (int j = r & 1; j + 1 < J; j += 2)
                if (key[j + 1] > key[j]) {
                    const uint32_t tk = key[j];
                    key[j] = key[j + 1];
                    key[j + 1] = tk;
                    const int tj = jo[j];
                    jo[j] = jo[j + 1];
                    jo[j + 1] = tj;
                }
        for (int k = 0; k < topk; ++k) {
            const uint32_t m = wave_max_u32(key[0]);
            const uint64_t hit = __ballot(key[0] == m);
            int e;
            if (__popcll(hit) == 1) {                                 // uniform: one lane holds the maximum
                const int wl = __ffsll((long long)hit) - 1;
                e = 64 * __builtin_amdgcn_readlane(jo[0], wl) + wl;
            } else {                                                  // equal keys: the lowest id
                e = (int)wave_min_u32(key[0] == m ? (uint32_t)(64 * jo[0] + lane) : 0xFFFFFFFFu);
            }
            if (lane == (e & 63)) {                                   // the winner's lane drops its best key
#pragma unroll
                for (int j = 0; j + 1 < J; ++j) {
                    key[j] = key[j + 1];
                    jo[j] = jo[j + 1];
                }
                key[J - 1] = 0u;
            }
            if (lane == k) mine_e = e;
        }
    } else {
        // many keys per lane: each round scans the lane's keys for its best (the lower j among equal keys)
        for (int k = 0; k < topk; ++k) {
            uint32_t bk = 0u;
            int bj = 0;
#pragma unroll
            for (int j = 0; j < J; ++j)
                if (key[j] > bk) {
                    bk = key[j];
                    bj = j;
                }
            const uint32_t m = wave_max_u32(bk);
            const uint64_t hit = __ballot(bk == m);
            int e;
            if (__popcll(hit) == 1) {
                const int wl = __ffsll((long long)hit) - 1;
                e = 64 * __builtin_amdgcn_readlane(bj, wl) + wl;
            } else {
                e = (int)wave_min_u32(bk == m ? (uint32_t)(64 * bj + lane) : 0xFFFFFFFFu);
            }
#pragma unroll
            for (int j = 0; j < J; ++j)
                if (j == (e >> 6) && lane == (e & 63)) key[j] = 0u;
            if (lane == k) mine_e = e;
        }
    }
    // scores of the picks (written by their owners before the rounds), summed in pick order
    const float mine = lane < topk ? sco[mine_e] : 0.f;
    float total = 0.f;
    for (int k = 0; k < topk; ++k)
        total = total + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mine), k));
    if (lane < topk) {
        float wv = mine;
        if (renorm) wv = __fdiv_rn(wv, total + 1e-20f);
        ids_row[lane] = mine_e;
        wts_row[lane] = wv * scale;
        ids_sh[lane] = mine_e;
        wts_sh[lane] = wv * scale;
    }
}

// One wave per token, four tokens per 256-thread workgroup: topk_wave over the token's logits (scores in LDS).
template <int J>
__global__ __launch_bounds__(256) void router_topk_kernel(const float* __restrict__ logits, int T, int E,
                                                          const float* __restrict__ bias, int topk, float scale,
                                                          int renorm, int32_t* __restrict__ ids,
                                                          float* __restrict__ wts) {
    __shared__ float sco[4 * 64 * J];
    __shared__ int ids_sh[4 * TOPK_MAX_K];
    __shared__ float wts_sh[4 * TOPK_MAX_K];
    const int wv = threadIdx.x >> 6;
    const int t = blockIdx.x * 4 + wv;
    if (t >= T) return;                                              // uniform over the wave (no block barrier)
    topk_wave<J>(logits + (size_t)t * E, E, bias, topk, scale, renorm, sco + wv * 64 * J, ids + (size_t)t * topk,
                 wts + (size_t)t * topk, ids_sh + wv * TOPK_MAX_K, wts_sh + wv * TOPK_MAX_K);
}

// The decode-size front end in one workgroup (P = T topk <= ROUTE_SMALL_MAX_P): wave w of the workgroup's nw takes
// the top-k of tokens w, w + nw, ...; then the whole permutation of route_small_body over the picks (int32 ids, fp32
// weights). The picks are written to global memory (the caller's copy) and to shared memory, from which the
// permutation reads them. Shared memory: the permutation's P + 2 (n + 1) ints, nw x E scores, then the picks' P ids
// and P weights.
template <int J, bool COH, bool SCORE = false>
__device__ __forceinline__ void topk_route_body(const float* __restrict__ logits, int T, int E,
                                                const float* __restrict__ bias, int topk, float scale, int renorm,
                                                int32_t* __restrict__ ids, float* __restrict__ wts, const RouteArgs& a,
                                                int* sh) {
    const int wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
    float* sco = reinterpret_cast<float*>(sh + a.P + 2 * (a.n + 1)) + wv * E;
    int* ids_sh = sh + a.P + 2 * (a.n + 1) + nw * E;
    float* wts_sh = reinterpret_cast<float*>(ids_sh + a.P);
    for (int t = wv; t < T; t += nw)
        topk_wave<J, COH, SCORE>(logits + (size_t)t * E, E, bias, topk, scale, renorm, sco, ids + (size_t)t * topk,
                          wts + (size_t)t * topk, ids_sh + t * topk, wts_sh + t * topk);
    __syncthreads();
    RouteArgs b = a;
    b.ids = ids_sh;
    b.w = wts_sh;
    b.wdt = DT_F32;
    if (a.P <= 64 && a.seg >= T) route_wave64<int32_t>(b);
    else route_small_body<int32_t>(b, sh);
}

// MAXT: the launch's threads (512 for J = 16, so that the sixteen keys per lane and their loads fit the registers)
template <int J, int MAXT = 1024>
__global__ __launch_bounds__(MAXT) void topk_route_kernel(const float* __restrict__ logits, int T, int E,
                                                          const float* __restrict__ bias, int topk, float scale,
                                                          int renorm, int32_t* __restrict__ ids,
                                                          float* __restrict__ wts, RouteArgs a) {
    extern __shared__ int sh[];
    topk_route_body<J, false>(logits, T, E, bias, topk, scale, renorm, ids, wts, a, sh);
}

constexpr int RR_EXPERTS = 2;   // router experts per workgroup of the one-launch front end (all in one round of CUs)
constexpr unsigned RR_GROUPS = 15;   // arrival groups (control words 64 (g + 1), g < 15, within a 4 KB control block)
// The whole decode-size front end in one launch: the router GEMV (RR_EXPERTS experts per workgroup, logits_body, which
// also applies the sigmoid so the ranking workgroup only loads scores), then the
// workgroup that finishes last (arrival counters at fixed workspace offsets, returned to zero by the arrivals that
// complete them) runs topk_route_body over all logits. Logits cross workgroups, and XCDs with their own L2, as
// device-coherent stores and loads; a workgroup arrives only after its stores have completed.
template <int J, int MAXT = 1024>
__global__ __launch_bounds__(MAXT) void router_route_kernel(const uint16_t* __restrict__ x, int64_t x_stride,
                                                            const uint16_t* __restrict__ w, int T, int K, int E,
                                                            float* __restrict__ logits, const float* __restrict__ bias,
                                                            int topk, float scale, int renorm,
                                                            int32_t* __restrict__ ids, float* __restrict__ wts,
                                                            RouteArgs a, unsigned* arrivals) {
    extern __shared__ int sh[];
    __shared__ int last;
    logits_body<true, RR_EXPERTS, true>(x, x_stride, w, T, K, E, RR_EXPERTS * blockIdx.x, logits);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    // the last of the grid's arrivals ranks. Two levels, so that no counter word queues more than ~16 atomics (one
    // word took ~8 ns per arrival): workgroup b counts on the word of its group b % G (words 64 (g + 1)), the group's
    // last arrival on word 0. Each count is taken modulo its number of arrivals, so that a counter left non-zero (a
    // workspace not zero-filled before its first use) still elects one workgroup per call and the tables are always
    // rebuilt; the last arrival of each level returns its word to zero.
    if (threadIdx.x == 0) {
        const unsigned G = min(RR_GROUPS, gridDim.x), g = blockIdx.x % G, size = (gridDim.x - 1 - g) / G + 1;
        unsigned* gw = arrivals + 64 * (g + 1);
        int l = 0;
        if ((__hip_atomic_fetch_add(gw, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u) % size == 0u) {
            __hip_atomic_store(gw, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            l = (__hip_atomic_fetch_add(arrivals, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u) % G == 0u;
        }
        last = l;
    }
    __syncthreads();
    if (!last) return;
    // no acquire fence: the only data other workgroups wrote here are the scores, stored device-coherent and complete
    // before their arrivals, and the ranking loads them device-coherent (from the coherence point, never from a line
    // this CU's or XCD's caches hold)
    if (threadIdx.x == 0) *arrivals = 0u;
    topk_route_body<J, true, true>(logits, T, E, bias, topk, scale, renorm, ids, wts, a, sh);
}

// Tables from pre-sorted pairs (the exl3_moe contract): counts [n+1] int64 give each expert's span of the sorted
// arrays; experts with 0 < count <= R get segments and pe = e on their span, every other row pe = -1; token ids
// outside [0, B) are skipped (pe = -1). code/fork/kernels/exl3.cu:529-566 (route_prep).
__global__ __launch_bounds__(1024) void route_counts_kernel(const int64_t* __restrict__ counts64,
                                                            const int64_t* __restrict__ token_sorted,
                                                            const uint16_t* __restrict__ weight_sorted, int B,
                                                            RouteArgs a) {
    extern __shared__ int sh[];
    __shared__ int tot[16];
    int* cnt = sh;
    int* start = sh + a.n;
    zero_counters(a);
    for (int j = threadIdx.x; j < a.P; j += blockDim.x) a.pe[j] = -1;
    int run = 0;
    for (int base = 0; base < a.n; base += blockDim.x) {
        const int e = base + threadIdx.x;
        const int64_t c64 = e < a.n ? counts64[e] : 0;
        const int c = c64 < 0 ? 0 : (c64 > a.P ? a.P + 1 : (int)c64);
        int ctot;
        const int cinc = block_scan_incl(c, tot, ctot);
        if (e < a.n) {
            const int st = run + cinc - c;
            start[e] = st;
            cnt[e] = (c > 0 && c <= a.R && st + c <= a.P) ? c : 0;    // ineligible experts: no rows, no segments
        }
        run += ctot;
    }
    __syncthreads();
    build_segments(cnt, start, a.n, a.R, a.seg, a.S_cap, a.seg_expert, a.seg_row0, a.seg_rows, a.nseg, tot);
    __syncthreads();
    for (int e = 0; e < a.n; ++e) {
        const int c = cnt[e], st = start[e];
        for (int i = threadIdx.x; i < c; i += blockDim.x) a.pe[st + i] = e;
    }
    __syncthreads();
    for (int j = threadIdx.x; j < a.P; j += blockDim.x) {
        const int64_t t = token_sorted[j];
        if (t < 0 || t >= B) {
            a.pe[j] = -1;
            a.tok[j] = 0;
        } else {
            a.tok[j] = (int)t;
        }
        a.w16[j] = weight_sorted[j];
    }
}

// Segment tables of rows grouped by expert (the e4m3 extension's seg_tables, code/fork/kernels/moe_e4m3.cu:2372-2400
// and :3066-3083): expert e's rows start at the exclusive scan of counts[0 .. n); every expert with rows gets
// ceil(count / tile) segments; num_rows = the total. One workgroup; n <= 4096.
__global__ __launch_bounds__(1024) void seg_tables_kernel(const int64_t* __restrict__ counts64, int n, int tile,
                                                          int max_segs, int* seg_expert, int* seg_row0, int* seg_rows,
                                                          int* nseg, int* nrows) {
    extern __shared__ int sh[];
    __shared__ int tot[16];
    int* cnt = sh;
    int* start = sh + n;
    int run = 0;
    for (int base = 0; base < n; base += blockDim.x) {
        const int e = base + threadIdx.x;
        const int64_t c64 = e < n ? counts64[e] : 0;
        const int c = c64 < 0 ? 0 : (c64 > (1 << 24) ? (1 << 24) : (int)c64);
        int ctot;
        const int cinc = block_scan_incl(c, tot, ctot);
        if (e < n) {
            cnt[e] = c;
            start[e] = run + cinc - c;
        }
        run += ctot;
    }
    __syncthreads();
    build_segments(cnt, start, n, 1 << 30, tile, max_segs, seg_expert, seg_row0, seg_rows, nseg, tot);
    if (threadIdx.x == 0) nrows[0] = run;
}

int launch_seg_tables(const int64_t* counts, int n, int tile, int max_segs, int* se, int* sr0, int* sr, int* ns,
                      int* nr, hipStream_t st) {
    hipLaunchKernelGGL(seg_tables_kernel, dim3(1), dim3(1024), (size_t)2 * n * sizeof(int), st, counts, n, tile,
                       max_segs, se, sr0, sr, ns, nr);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Row tables of the grouped tier's fat experts (the contract of code/fork/docs/prod_exl3_reference.py:1316-1361): the
// experts with more than `cap` pairs (counts int64 [n], the pairs sorted by expert) laid out back to back in expert
// order, segments of at most `tile` rows. fat_scan_kernel (one workgroup): the exclusive scans of the counts (each
// expert's first sorted position) and of the fat counts (its first row), the segment table (build_segments with the
// thin experts excluded), num_rows, and per expert (first row, first sorted position) into sc [2 n].
__global__ __launch_bounds__(1024) void fat_scan_kernel(const int64_t* __restrict__ counts64, int n, int cap, int tile,
                                                        int max_segs, int* seg_expert, int* seg_row0, int* seg_rows,
                                                        int* nseg, int* nrows, int* sc) {
    extern __shared__ int sh[];
    __shared__ int tot[16];
    int* cnt = sh;
    int* row0 = sh + n;
    int run = 0, frun = 0;
    for (int base = 0; base < n; base += blockDim.x) {
        const int e = base + threadIdx.x;
        const int64_t c64 = e < n ? counts64[e] : 0;
        const int c = c64 < 0 ? 0 : (c64 > (1 << 24) ? (1 << 24) : (int)c64);
        const int f = c > cap ? c : 0;
        int ctot, ftot;
        const int cinc = block_scan_incl(c, tot, ctot);
        const int finc = block_scan_incl(f, tot, ftot);
        if (e < n) {
            cnt[e] = c;
            row0[e] = frun + finc - f;
            sc[e] = row0[e];
            sc[n + e] = run + cinc - c;
        }
        run += ctot;
        frun += ftot;
    }
    __syncthreads();
    build_segments(cnt, row0, n, 1 << 30, tile, max_segs, seg_expert, seg_row0, seg_rows, nseg, tot, cap);
    if (threadIdx.x == 0) nrows[0] = frun;
}

// fat_rows_kernel: workgroup e < n writes the rows of fat expert e (row sc[e] + i = sorted position sc[n + e] + i: its
// token and weight, and e); the workgroups past n mark the rows no fat expert fills (expert -1, token 0, weight 0).
// Rows past rows_cap and sorted positions past the arrays (inconsistent counts) are left out.
__global__ __launch_bounds__(256) void fat_rows_kernel(const int64_t* __restrict__ counts64, int n, int cap,
                                                       const int64_t* __restrict__ token_sorted,
                                                       const uint16_t* __restrict__ weight_sorted, int rows_cap,
                                                       const int* __restrict__ sc, const int* __restrict__ nrows,
                                                       int* row_expert, int64_t* row_token, uint16_t* row_weight) {
    const int b = blockIdx.x;
    if (b < n) {
        const int64_t c = counts64[b];
        if (c <= cap) return;
        const int r0 = sc[b], p0 = sc[n + b];
        for (int i = threadIdx.x; i < c; i += 256) {
            const int r = r0 + i, p = p0 + i;
            if (r >= rows_cap || p >= rows_cap) break;
            row_expert[r] = b;
            row_token[r] = token_sorted[p];
            row_weight[r] = weight_sorted[p];
        }
        return;
    }
    for (int r = nrows[0] + (b - n) * 256 + threadIdx.x; r < rows_cap; r += (gridDim.x - n) * 256) {
        row_expert[r] = -1;
        row_token[r] = 0;
        row_weight[r] = 0;
    }
}

int launch_fat_tables(const int64_t* counts, int n, int cap, const int64_t* token_sorted,
                      const uint16_t* weight_sorted, int rows_cap, int tile, int max_segs, int* se, int* sr0, int* sr,
                      int* ns, int* nr, int* row_expert, int64_t* row_token, uint16_t* row_weight, int* sc,
                      hipStream_t st) {
    hipLaunchKernelGGL(fat_scan_kernel, dim3(1), dim3(1024), (size_t)2 * n * sizeof(int), st, counts, n, cap, tile,
                       max_segs, se, sr0, sr, ns, nr, sc);
    const int tail = std::max(1, std::min(1024, (rows_cap + 255) / 256));
    hipLaunchKernelGGL(fat_rows_kernel, dim3(n + tail), dim3(256), 0, st, counts, n, cap, token_sorted, weight_sorted,
                       rows_cap, sc, nr, row_expert, row_token, row_weight);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// The e4m3 extension's plan tables (code/fork/overlay/glm53_moe_e4m3.py:450-477) from a permutation of the routed
// pairs (launch_route: sorted by local id, sentinel pairs last, pe = -1 for them): per sorted position p the row's
// token, fp32 weight and local expert (n for the sentinel rows); per pair j its row inv[j] and its local id; the
// counts [n + 1] widened to int64.
__global__ __launch_bounds__(256) void route_rows_kernel(RouteArgs a, int* local, int* pos, int64_t* row_token,
                                                         float* row_weight, int* row_expert, int64_t* counts64) {
    for (int i = blockIdx.x * 256 + threadIdx.x; i < max(a.P, a.n + 1); i += gridDim.x * 256) {
        if (i < a.P) {
            const int e = a.pe[i];
            row_token[i] = a.tok[i];
            row_weight[i] = a.w32[i];
            row_expert[i] = e >= 0 ? e : a.n;
            const int p = a.inv[i];
            const int ep = a.pe[p];
            pos[i] = p;
            local[i] = ep >= 0 ? ep : a.n;
        }
        if (i <= a.n) counts64[i] = a.counts[i];
    }
}

int launch_route_rows(const RouteArgs& a, int* local, int* pos, int64_t* row_token, float* row_weight,
                      int* row_expert, int64_t* counts64, hipStream_t st) {
    if (launch_route(a, st)) return -1;
    const int g = std::max(1, std::min(1024, (std::max(a.P, a.n + 1) + 255) / 256));
    hipLaunchKernelGGL(route_rows_kernel, dim3(g), dim3(256), 0, st, a, local, pos, row_token, row_weight, row_expert,
                       counts64);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Multi-block permutation for large P: (1) per-block counts, (2) one block scans them into per-block offsets
// and builds the segments, (3) every block places its pairs (rank inside the block by pair index).
constexpr int ROUTE_BLK = 1024;

template <typename IT>
__global__ __launch_bounds__(ROUTE_BLK) void route_hist_kernel(RouteArgs a) {
    extern __shared__ int cnt[];
    const IT* ids = reinterpret_cast<const IT*>(a.ids);
    zero_counters(a);
    for (int e = threadIdx.x; e <= a.n; e += blockDim.x) cnt[e] = 0;
    __syncthreads();
    const int j = blockIdx.x * ROUTE_BLK + threadIdx.x;
    if (j < a.P) {
        const int l = local_id<IT>(ids[j], a.emap, a.n_global, a.n);
        a.loc[j] = l;
        atomicAdd(&cnt[l], 1);
    }
    __syncthreads();
    for (int e = threadIdx.x; e <= a.n; e += blockDim.x) a.blk_cnt[(size_t)blockIdx.x * (a.n + 1) + e] = cnt[e];
}

__global__ __launch_bounds__(1024) void route_scan_kernel(RouteArgs a, int nblk) {
    extern __shared__ int sh[];
    __shared__ int tot[16];
    int* cnt = sh;
    int* start = sh + (a.n + 1);
    for (int e = threadIdx.x; e <= a.n; e += blockDim.x) {
        int c = 0;
        for (int b = 0; b < nblk; ++b) c += a.blk_cnt[(size_t)b * (a.n + 1) + e];
        cnt[e] = c;
    }
    __syncthreads();
    int run = 0;
    for (int base = 0; base <= a.n; base += blockDim.x) {
        const int e = base + threadIdx.x;
        const int c = e <= a.n ? cnt[e] : 0;
        int ctot;
        const int cinc = block_scan_incl(c, tot, ctot);
        if (e <= a.n) start[e] = run + cinc - c;
        run += ctot;
    }
    __syncthreads();
    for (int e = threadIdx.x; e <= a.n; e += blockDim.x) {
        int off = start[e];
        for (int b = 0; b < nblk; ++b) {
            const size_t i = (size_t)b * (a.n + 1) + e;
            const int c = a.blk_cnt[i];
            a.blk_cnt[i] = off;
            off += c;
        }
        if (a.counts) a.counts[e] = cnt[e];
        a.cnt_out[e] = cnt[e];
    }
    build_segments(cnt, start, a.n, a.R, a.seg, a.S_cap, a.seg_expert, a.seg_row0, a.seg_rows, a.nseg, tot, a.Rmin);
}

// route_scan_kernel with the per-block counts staged in LDS (nblk <= 64 blocks, (n + 1) * nblk ints): one coalesced
// read of blk_cnt, the scans over blocks in LDS (one wave per local id, lane = block), one coalesced write of the
// offsets, so no global load waits on a store. Same tables as route_scan_kernel.
constexpr size_t ROUTE_SCAN_LDS_MAX = 120 * 1024;
__global__ __launch_bounds__(1024) void route_scan_lds_kernel(RouteArgs a, int nblk) {
    extern __shared__ int sh[];
    __shared__ int tot[16];
    const int n1 = a.n + 1, cells = n1 * nblk;
    int* cnt = sh;
    int* start = sh + n1;
    int* stage = sh + 2 * n1;                                         // [nblk][n1]
    for (int i = threadIdx.x; i < cells; i += blockDim.x) stage[i] = a.blk_cnt[i];
    __syncthreads();
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
    for (int e = wv; e < n1; e += nw) {
        const int v = lane < nblk ? stage[lane * n1 + e] : 0;
        const int incl = wave_scan_incl(v);
        if (lane < nblk) stage[lane * n1 + e] = incl - v;             // this id's pairs in earlier blocks
        if (lane == 63) cnt[e] = incl;
    }
    __syncthreads();
    int run = 0;
    for (int base = 0; base <= a.n; base += blockDim.x) {
        const int e = base + threadIdx.x;
        const int c = e <= a.n ? cnt[e] : 0;
        int ctot;
        const int cinc = block_scan_incl(c, tot, ctot);
        if (e <= a.n) start[e] = run + cinc - c;
        run += ctot;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < cells; i += blockDim.x) a.blk_cnt[i] = start[i % n1] + stage[i];
    for (int e = threadIdx.x; e <= a.n; e += blockDim.x) {
        if (a.counts) a.counts[e] = cnt[e];
        a.cnt_out[e] = cnt[e];
    }
    build_segments(cnt, start, a.n, a.R, a.seg, a.S_cap, a.seg_expert, a.seg_row0, a.seg_rows, a.nseg, tot, a.Rmin);
}

// route_place_kernel with the ranks from ballots (n + 1 <= ROUTE_MATCH_MAX_IDS): in each wave the lanes holding the
// same id are the AND over the id's bits of the ballots of lanes agreeing on that bit, so a lane's rank in its wave
// is a popcount; the earlier waves' pairs of an id come from per-wave counts (written by each id's first lane) summed
// in wave order. Same ranks as route_place_kernel (pairs of an id in pair-index order), without its O(block) scan.
constexpr int ROUTE_MATCH_MAX_IDS = 1024;
__global__ __launch_bounds__(ROUTE_BLK) void route_place_match_kernel(RouteArgs a) {
    extern __shared__ int wh[];                                       // [ROUTE_BLK / 64 waves][n + 1]
    constexpr int NW = ROUTE_BLK / 64;
    const int n1 = a.n + 1;
    const int j0 = blockIdx.x * ROUTE_BLK;
    const int j = j0 + threadIdx.x;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const bool valid = j < a.P;
    for (int i = threadIdx.x; i < NW * n1; i += ROUTE_BLK) wh[i] = 0;
    const int l = valid ? a.loc[j] : 0;
    uint64_t same = __ballot(valid);
    const int nbits = 32 - __builtin_clz((unsigned)max(a.n, 1));       // ids 0 .. n
    for (int b = 0; b < nbits; ++b) {
        const bool bit = (l >> b) & 1;
        const uint64_t m = __ballot(bit);
        same &= bit ? m : ~m;
    }
    const int wrank = __popcll(same & ((1ull << lane) - 1));
    __syncthreads();                                                  // (the zeroed counts)
    if (valid && wrank == 0) wh[wv * n1 + l] = __popcll(same);
    __syncthreads();
    for (int e = threadIdx.x; e < n1; e += ROUTE_BLK) {               // counts -> earlier waves' pairs of id e
        int run = 0;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const int c = wh[w * n1 + e];
            wh[w * n1 + e] = run;
            run += c;
        }
    }
    __syncthreads();
    if (!valid) return;
    const int pos = a.blk_cnt[(size_t)blockIdx.x * n1 + l] + wh[wv * n1 + l] + wrank;
    a.tok[pos] = j / a.topk;
    a.w16[pos] = weight_f16(a.w, a.wdt, j);
    if (a.w32) a.w32[pos] = weight_f32(a.w, a.wdt, j);
    a.pe[pos] = (l < a.n && a.cnt_out[l] <= a.R && a.cnt_out[l] > a.Rmin) ? l : -1;
    a.inv[j] = pos;
}

__global__ __launch_bounds__(ROUTE_BLK) void route_place_kernel(RouteArgs a) {
    __shared__ __align__(16) int loc[ROUTE_BLK];
    const int j0 = blockIdx.x * ROUTE_BLK;
    const int j = j0 + threadIdx.x;
    const int nj = min(ROUTE_BLK, a.P - j0);
    if (threadIdx.x < nj) loc[threadIdx.x] = a.loc[j];
    __syncthreads();
    if (threadIdx.x >= nj) return;
    const int l = loc[threadIdx.x];
    // rank among the block's earlier pairs with the same id: the earlier waves' pairs (a bound uniform over the
    // wave, four per LDS read), then this wave's earlier lanes
    const int w0 = threadIdx.x & ~63;
    const int4* l4 = reinterpret_cast<const int4*>(loc);
    int rank = 0;
#pragma unroll 8
    for (int i4 = 0; i4 < (w0 >> 2); ++i4) {
        const int4 v = l4[i4];
        rank += (v.x == l) + (v.y == l) + (v.z == l) + (v.w == l);
    }
    const int me = threadIdx.x;
#pragma unroll
    for (int i4 = w0 >> 2; i4 < (w0 >> 2) + 16; ++i4) {
        const int4 v = l4[i4];
        const int i = 4 * i4;
        rank += (i < me && v.x == l) + (i + 1 < me && v.y == l) + (i + 2 < me && v.z == l) + (i + 3 < me && v.w == l);
    }
    const int pos = a.blk_cnt[(size_t)blockIdx.x * (a.n + 1) + l] + rank;
    a.tok[pos] = j / a.topk;
    a.w16[pos] = weight_f16(a.w, a.wdt, j);
    if (a.w32) a.w32[pos] = weight_f32(a.w, a.wdt, j);
    a.pe[pos] = (l < a.n && a.cnt_out[l] <= a.R && a.cnt_out[l] > a.Rmin) ? l : -1;
    a.inv[j] = pos;
}

// ------------------------------------------------------------------------------------------------ launchers

int launch_router_logits(const uint16_t* x, int64_t x_stride, const uint16_t* w, int T, int K, int E, float* logits,
                         hipStream_t st) {
    if (T >= RG_MIN_T) {
        const int64_t waves = (int64_t)((T + RG_TOK - 1) / RG_TOK) * ((E + RG_EXP - 1) / RG_EXP);
        hipLaunchKernelGGL(router_gemm_f64_kernel, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, x, x_stride, w,
                           T, K, E, logits);
    } else {
        hipLaunchKernelGGL(router_logits_kernel, dim3(E), dim3(64 * (K / 512)), 0, st, x, x_stride, w, T, K, E,
                           logits);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_router_topk(const float* logits, int T, int E, const float* bias, int topk, float scale, int renorm,
                       int32_t* ids, float* wts, hipStream_t st) {
    if (E > TOPK_MAX_E || topk > TOPK_MAX_K) return -1;
    const dim3 g((T + 3) / 4);
    if (T <= 0) return 0;
    if (E <= 320) hipLaunchKernelGGL(router_topk_kernel<5>, g, dim3(256), 0, st, logits, T, E, bias, topk, scale, renorm, ids, wts);
    else hipLaunchKernelGGL(router_topk_kernel<16>, g, dim3(256), 0, st, logits, T, E, bias, topk, scale, renorm, ids, wts);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_topk_route(const float* logits, int T, int E, const float* bias, int topk, float scale, int renorm,
                      int32_t* ids, float* wts, const RouteArgs& a, hipStream_t st) {
    if (a.P > ROUTE_SMALL_MAX_P || a.ids64 || a.ids != ids || E > TOPK_MAX_E) return -1;
    const size_t shm = (size_t)(3 * a.P + 2 * (a.n + 1)) * sizeof(int) + (size_t)16 * E * sizeof(float);
    static bool attr = false;                                         // up to 45 KB + 64 KB for E = 1024
    if (!attr) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(topk_route_kernel<16, 512>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, 128 * 1024) != hipSuccess)
            return -1;
        attr = true;
    }
    if (E <= 320)
        hipLaunchKernelGGL(topk_route_kernel<5>, dim3(1), dim3(1024), shm, st, logits, T, E, bias, topk, scale, renorm,
                           ids, wts, a);
    else
        hipLaunchKernelGGL((topk_route_kernel<16, 512>), dim3(1), dim3(512), shm, st, logits, T, E, bias, topk, scale,
                           renorm, ids, wts, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_router_route(const uint16_t* x, int64_t x_stride, const uint16_t* w, int K, float* logits, int T, int E,
                        const float* bias, int topk, float scale, int renorm, int32_t* ids, float* wts,
                        const RouteArgs& a, unsigned* arrivals, hipStream_t st) {
    if (a.P > ROUTE_SMALL_MAX_P || a.ids64 || a.ids != ids || E > TOPK_MAX_E || K % 512 || K / 512 > RL_MAXC) return -1;
    const int nw = K / 512;
    const size_t shm = (size_t)(3 * a.P + 2 * (a.n + 1)) * sizeof(int) + (size_t)nw * E * sizeof(float);
    static bool attr = false;
    if (!attr) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(router_route_kernel<16>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, 128 * 1024) != hipSuccess ||
            hipFuncSetAttribute(reinterpret_cast<const void*>(router_route_kernel<16, 512>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, 128 * 1024) != hipSuccess)
            return -1;
        attr = true;
    }
    const dim3 grid((E + RR_EXPERTS - 1) / RR_EXPERTS);
    if (E <= 320)
        hipLaunchKernelGGL(router_route_kernel<5>, grid, dim3(64 * nw), shm, st, x, x_stride, w, T, K, E, logits,
                           bias, topk, scale, renorm, ids, wts, a, arrivals);
    else if (nw <= 8)                                                 // K <= 4096: at most 512 threads
        hipLaunchKernelGGL((router_route_kernel<16, 512>), grid, dim3(64 * nw), shm, st, x, x_stride, w, T, K, E,
                           logits, bias, topk, scale, renorm, ids, wts, a, arrivals);
    else
        hipLaunchKernelGGL(router_route_kernel<16>, grid, dim3(64 * nw), shm, st, x, x_stride, w, T, K, E, logits,
                           bias, topk, scale, renorm, ids, wts, a, arrivals);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_route_counts(const int64_t* counts64, const int64_t* token_sorted, const uint16_t* weight_sorted, int B,
                        const RouteArgs& a, hipStream_t st) {
    const size_t shm = (size_t)2 * a.n * sizeof(int);
    hipLaunchKernelGGL(route_counts_kernel, dim3(1), dim3(1024), shm, st, counts64, token_sorted, weight_sorted, B, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_route(const RouteArgs& a, hipStream_t st) {
    if (a.P <= ROUTE_SMALL_MAX_P) {
        const size_t shm = (size_t)(a.P + 2 * (a.n + 1)) * sizeof(int);
        if (a.ids64) hipLaunchKernelGGL(route_small_kernel<int64_t>, dim3(1), dim3(1024), shm, st, a);
        else hipLaunchKernelGGL(route_small_kernel<int32_t>, dim3(1), dim3(1024), shm, st, a);
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    const int nblk = (a.P + ROUTE_BLK - 1) / ROUTE_BLK;
    const size_t shm1 = (size_t)(a.n + 1) * sizeof(int);
    if (a.ids64) hipLaunchKernelGGL(route_hist_kernel<int64_t>, dim3(nblk), dim3(ROUTE_BLK), shm1, st, a);
    else hipLaunchKernelGGL(route_hist_kernel<int32_t>, dim3(nblk), dim3(ROUTE_BLK), shm1, st, a);
    const size_t shm_lds = (size_t)(a.n + 1) * (2 + nblk) * sizeof(int);
    static bool lds_attr = false;
    if (nblk <= 64 && shm_lds <= ROUTE_SCAN_LDS_MAX && !lds_attr) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(route_scan_lds_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)ROUTE_SCAN_LDS_MAX) != hipSuccess)
            return -1;
        lds_attr = true;
    }
    if (nblk <= 64 && shm_lds <= ROUTE_SCAN_LDS_MAX)
        hipLaunchKernelGGL(route_scan_lds_kernel, dim3(1), dim3(1024), shm_lds, st, a, nblk);
    else
        hipLaunchKernelGGL(route_scan_kernel, dim3(1), dim3(1024), 2 * shm1, st, a, nblk);
    if (a.n + 1 <= ROUTE_MATCH_MAX_IDS)
        hipLaunchKernelGGL(route_place_match_kernel, dim3(nblk), dim3(ROUTE_BLK),
                           (size_t)(ROUTE_BLK / 64) * (a.n + 1) * sizeof(int), st, a);
    else
        hipLaunchKernelGGL(route_place_kernel, dim3(nblk), dim3(ROUTE_BLK), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace mi355moe
