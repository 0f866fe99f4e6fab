// Prefill-path kernels (many rows per expert, the E3 grouped tier): gather + input rotation, the gate/up grouped
// GEMM and the down grouped GEMM on fp16 MFMA (v_mfma_f32_32x32x16_f16) with the EXL3 trellis decoded into LDS.
//
// Tiles: a workgroup of 8 waves owns a 256-row segment of one expert (rows sorted by expert) and one column block:
//   gate/up: 128 columns of gate and the same 128 of up (waves 2g and 2g+1: rows 64g..64g+63 of gate / of up);
//   down:    256 output columns (two 128-column halves).
// Per K step of 32: every thread loads 8 bytes of trellis (two words of one 16x16 tile) and 32 bytes of the A rows
// for the next step while the MFMAs of the current step run; the decoded B step (32 k x 256 columns fp16) and the A
// step (256 rows x 32 k fp16) are double-buffered in LDS. Each weight value is decoded once per 256-row tile.
// Numerics (oracle/csrc/oracle.c mode 1 = the E3 kernels, code/fork/docs/ref/mia_exl3-fat-kernel/exl3_fat_moe.cu):
//   gather   h13 = fp16(H(fp16(x * suh_g)) * r)                                         (exl3_fat_moe.cu:95-126)
//   gate/up  g = (H(acc_g) * r) * svh_g, u likewise; iff L != 0: g = min(g, L), u = clamp(u, -L, L);
//            a = (1 / (1 + (float)exp(-(double)g))) * g * u; h2 = fp16(H(fp16(fp16(a) * suh_d)) * r)  (:340-378)
//   down     contribution ((H(acc_d) * r) * svh_d) * w16 per pair                       (:443-457); out[token] =
//            the token's contributions summed in slot order (fp32), then the output dtype
#include <algorithm>

#include "common.cuh"
#include "mi355moe_internal.h"

namespace mi355moe {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));

constexpr int PF_TM = PREFILL_TM;   // rows per tile (segment height)
constexpr int PF_THREADS = 512;     // 8 waves
constexpr int PF_LD = 40;           // halves per LDS row of a decoded B step (32 k + 8 padding)
constexpr int PF_NS = 4;            // staged steps in flight (A rows and raw trellis words)
constexpr int PF_ASB = PF_TM * 64;              // one A stage: 256 rows x 32 k fp16, bytes
constexpr int PF_WSB = 4096;                    // one raw-word stage: 2 halves x 2 k tiles x 8 column tiles x 128 B
constexpr int PF_BS = 2 * 128 * PF_LD;          // one decoded B stage: 2 x 128 columns (halves)
constexpr size_t PF_LDS = (size_t)PF_NS * (PF_ASB + PF_WSB) + (size_t)2 * PF_BS * 2;   // 122,880 bytes

// ------------------------------------------------------------------------------------------------ gather

// h13[pos] = rotated x[tok[pos]] with expert pe[pos]'s gate suh, for every row with pe >= 0; one wave per
// (row, 128-block) task, grid-stride.
__global__ __launch_bounds__(256) void pf_gather_kernel(PrefillArgs a) {
    const int lane = threadIdx.x & 63;
    const int nb = a.K >> 7;
    const int64_t tasks = (int64_t)a.P * nb;
    for (int64_t task = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); task < tasks; task += (int64_t)gridDim.x * 4) {
        const int pos = (int)(task / nb), blk = (int)(task - (int64_t)pos * nb);
        const int e = a.pe[pos];
        if (e < 0) continue;
        const _Float16* suh = reinterpret_cast<const _Float16*>(a.wt.g_suh[e]) + blk * 128;
        const size_t xoff = (size_t)a.tok[pos] * a.x_stride + blk * 128;
        _Float16 h0, h1;
        if (a.xdt == DT_BF16) {
            const uint32_t v = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint16_t*>(a.x) + xoff +
                                                                   2 * lane);
            h0 = (_Float16)__builtin_bit_cast(float, v << 16);
            h1 = (_Float16)__builtin_bit_cast(float, v & 0xFFFF0000u);
        } else {
            const h2 v = *reinterpret_cast<const h2*>(reinterpret_cast<const uint16_t*>(a.x) + xoff + 2 * lane);
            h0 = v.x;
            h1 = v.y;
        }
        const h2 s = *reinterpret_cast<const h2*>(suh + 2 * lane);
        float p0 = (float)(_Float16)(h0 * s.x), p1 = (float)(_Float16)(h1 * s.y);
        fwht128_w64(p0, p1, lane);
        *reinterpret_cast<h2*>(reinterpret_cast<_Float16*>(a.h13) + (size_t)pos * a.K + blk * 128 + 2 * lane) =
            h2{(_Float16)(p0 * HAD_R), (_Float16)(p1 * HAD_R)};
    }
}

// ------------------------------------------------------------------------------------------------ GEMM core

// Decode this thread's two trellis words (words 2wp, 2wp+1 of one tile, pw = word 2wp - 1 mod 32) into the B
// stage: column-major [col][k] with the k of the 32-step contiguous.
__device__ __forceinline__ void pf_store_b(uint32_t pw0, uint32_t w0, uint32_t w1, int wp, _Float16* B, int col_base,
                                           int krow) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t w = i ? w1 : w0;
        const uint32_t pw = i ? w0 : pw0;
        const int l = 2 * wp + i;
        h2 d[4];
        decode_word(pw, w, d);
        const int c0 = col_base + (l >> 2), r0 = krow + 2 * (l & 3);
        *reinterpret_cast<h2*>(B + c0 * PF_LD + r0) = d[0];
        *reinterpret_cast<h2*>(B + c0 * PF_LD + r0 + 8) = d[1];
        *reinterpret_cast<h2*>(B + (c0 + 8) * PF_LD + r0) = d[2];
        *reinterpret_cast<h2*>(B + (c0 + 8) * PF_LD + r0 + 8) = d[3];
    }
}

// The tile GEMM: acc[rb][c4] (32x32 blocks) of rows 64*rg + 32*rb, columns 32*c4 of B half `half` (128 columns),
// over kdim. A rows come from `a_rows` (row stride kdim), clamped to rn - 1. B tiles: (k tile, column tile) ->
// trellis words of matrix `bmat[half]` at ((kt * btiles_n) + bcol0[half] + ct) * 32.
struct PfTile {
    const uint16_t* a_rows;       // first row of the segment
    int rn, kdim;
    const uint32_t* btr[2];       // trellis of half 0 / 1
    int btiles_n;                 // tiles per trellis row (the matrix's column tiles)
    int bcol0[2];                 // first column tile of half 0 / 1
};

// A stage row R: 64 bytes = four 16-byte chunks (k 0-7, 8-15, 16-23, 24-31), chunk g at slot g ^ pf_swz(R): the
// fragment reads (16 consecutive rows per LDS pass, one chunk each) then touch every bank once.
__device__ __forceinline__ int pf_swz(int R) { return (R >> 2) & 3; }

// Staging, PF_NS steps deep, entirely by LDS DMA (global_load_lds): per 32-k step every wave copies 32 A rows (two
// 1 KB instructions: 16 rows x 4 chunks, swizzled through the source addresses) and a quarter of the step's raw
// trellis words (two 256-byte instructions). Step it + PF_NS - 1 is issued while step it is multiplied, so each
// load has PF_NS - 1 steps of MFMA work to arrive; loads past the last step re-read it. The decoded B stage of step
// it + 1 is built from its raw words during step it (double-buffered), so the decode arithmetic runs beside the
// MFMAs. One wait + barrier per step publishes A(it) and the raw words of step it + 1.
__device__ __forceinline__ void pf_gemm(const PfTile& t, unsigned char* smem, f16v (&acc)[2][4]) {
    unsigned char* Ast = smem;                                        // [PF_NS][256 rows][64 B]
    unsigned char* Wst = smem + PF_NS * PF_ASB;                       // [PF_NS][4 KB]
    _Float16* Bs = reinterpret_cast<_Float16*>(Wst + PF_NS * PF_WSB); // [2][2 halves][128 cols][PF_LD]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rg = wv >> 1, half = wv & 1;
    const int steps = t.kdim / 32;
    // A DMA sources: instruction i of this wave = rows 32 wv + 16 i + lane / 4, slot lane % 4
    const uint16_t* asrc[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int R = 32 * wv + 16 * i + (lane >> 2);
        const int chunk = (lane & 3) ^ pf_swz(R);
        asrc[i] = t.a_rows + (size_t)min(R, t.rn - 1) * t.kdim + 8 * chunk;
    }
    // raw-word DMA sources: instruction i of this wave = 256-byte part p of block (half hb, k tile kb)
    const uint32_t* wsrc[2];
    int wdst[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int ins = 2 * wv + i, blk = ins >> 2, part = ins & 3, hb = blk >> 1, kb = blk & 1;
        wsrc[i] = t.btr[hb] + ((size_t)kb * t.btiles_n + t.bcol0[hb]) * 32 + part * 64 + lane;
        wdst[i] = blk * 1024 + part * 256;
    }
    const size_t wstep = (size_t)2 * t.btiles_n * 32;                 // words per step (two k tiles)
    auto issue = [&](int sa, int sw) {                                // A of step sa, raw words of step sw (clamped)
        sa = min(sa, steps - 1);
        sw = min(sw, steps - 1);
        unsigned char* ad = Ast + (sa % PF_NS) * PF_ASB + wv * 2048;
#pragma unroll
        for (int i = 0; i < 2; ++i) dma16(asrc[i] + (size_t)sa * 32, ad + i * 1024);
        unsigned char* wd = Wst + (sw % PF_NS) * PF_WSB;
#pragma unroll
        for (int i = 0; i < 2; ++i) dma4(wsrc[i] + (size_t)sw * wstep, wd + wdst[i]);
    };
    // decoder role of this thread: half bm, tile bt (k tile bkt, column tile bct), word pair wp
    const int bm = tid >> 8, bt = (tid >> 4) & 15, bkt = bt >> 3, bct = bt & 7, wp = tid & 15;
    const int wofs = ((bm * 2 + bkt) * 8 + bct) * 128;               // the tile's 128 bytes in a raw-word stage
    auto decode = [&](int sw, int bb) {                               // raw words of step sw -> decoded stage bb
        const unsigned char* ws = Wst + (sw % PF_NS) * PF_WSB + wofs;
        const uint2 w = *reinterpret_cast<const uint2*>(ws + 8 * wp);
        const uint32_t pw = *reinterpret_cast<const uint32_t*>(ws + 4 * ((2 * wp + 31) & 31));
        pf_store_b(pw, w.x, w.y, wp, Bs + bb * PF_BS + bm * 128 * PF_LD, bct * 16, bkt * 16);
    };
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[rb][c][r] = 0.f;
    // prologue: raw words of step 0 first, then the batches that step it = 0, 1, 2 of the loop would have issued
    // (A(0..PF_NS-2), words(1..PF_NS-1)); decode step 0
    {
        unsigned char* wd = Wst;
#pragma unroll
        for (int i = 0; i < 2; ++i) dma4(wsrc[i], wd + wdst[i]);
    }
#pragma unroll
    for (int j = 0; j < PF_NS - 1; ++j) issue(j, j + 1);
    WAIT_VM(4 * (PF_NS - 1));                                         // the step-0 words
    LDS_BARRIER();
    decode(0, 0);
    for (int it0 = 0; it0 < steps; it0 += PF_NS) {
#pragma unroll
        for (int j = 0; j < PF_NS; ++j) {
            const int it = it0 + j;
            WAIT_VM(4 * (PF_NS - 2));                                 // A(it) and words(it + 1): the oldest batch
            LDS_BARRIER();
            issue(it + PF_NS - 1, it + PF_NS);
            const unsigned char* as = Ast + j * PF_ASB;               // it % PF_NS == j
            const _Float16* bs = Bs + (j & 1) * PF_BS + half * 128 * PF_LD;
#pragma unroll
            for (int kh = 0; kh < 2; ++kh) {
                h8 af[2], bf[4];
#pragma unroll
                for (int rb = 0; rb < 2; ++rb) {
                    const int R = 64 * rg + 32 * rb + (lane & 31);
                    const int slot = (2 * kh + (lane >> 5)) ^ pf_swz(R);
                    af[rb] = *reinterpret_cast<const h8*>(as + R * 64 + 16 * slot);
                }
                const int k = 16 * kh + 8 * (lane >> 5);
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    bf[c] = *reinterpret_cast<const h8*>(bs + (32 * c + (lane & 31)) * PF_LD + k);
#pragma unroll
                for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        acc[rb][c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[rb], bf[c], acc[rb][c], 0, 0, 0);
            }
            decode(it + 1, (j + 1) & 1);                              // step it + 1 (past the end: never used)
        }
    }
    WAIT_VM(0);                                                       // nothing in flight when LDS is reused
    LDS_BARRIER();
}

// Stage the accumulators of row block (rg2, rb) (32 rows x 256 columns) into Cs [32][256] fp32.
__device__ __forceinline__ void pf_stage_rows(const f16v (&acc)[2][4], float* Cs, int rg2, int rb) {
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if ((wv >> 1) != rg2) return;
    const int half = wv & 1;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            Cs[row * 256 + half * 128 + 32 * c + (lane & 31)] = acc[rb][c][r];
        }
}

// ------------------------------------------------------------------------------------------------ tile order

// Tile (segment s, column block cb) of 1D workgroup b: consecutive workgroups are dealt round-robin to the 8 XCDs
// (b % 8), so XCD x runs segments x, x + 8, x + 16, ... with all ncb column blocks of a segment in a row. The
// column blocks of one segment therefore share the XCD's L2 for their common A rows (read from HBM once per
// segment instead of once per column block). Grid: 8 * ncb * ceil(S_cap / 8).
__device__ __forceinline__ void pf_tile_of(int b, int ncb, int& s, int& cb) {
    const int x = b & 7, q = b >> 3;
    cb = q % ncb;
    s = 8 * (q / ncb) + x;
}

// ------------------------------------------------------------------------------------------------ gate/up

__global__ __launch_bounds__(PF_THREADS, 1) void pf_gateup_kernel(PrefillArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    int s, cb;
    pf_tile_of(blockIdx.x, a.N >> 7, s, cb);
    if (s >= a.nseg[0]) return;
    const int e = a.seg_expert[s], row0 = a.seg_row0[s], rn = a.seg_rows[s];
    const int K = a.K, N = a.N;
    PfTile t;
    t.a_rows = a.h13 + (size_t)row0 * K;
    t.rn = rn;
    t.kdim = K;
    t.btr[0] = reinterpret_cast<const uint32_t*>(a.wt.g_tr[e]);
    t.btr[1] = reinterpret_cast<const uint32_t*>(a.wt.u_tr[e]);
    t.btiles_n = N >> 4;
    t.bcol0[0] = t.bcol0[1] = cb * 8;
    f16v acc[2][4];
    pf_gemm(t, smem, acc);

    float* Cs = reinterpret_cast<float*>(smem);
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = cb * 128 + 2 * lane;
    const h2 svg = *reinterpret_cast<const h2*>(reinterpret_cast<const _Float16*>(a.wt.g_svh[e]) + col);
    const h2 svu = *reinterpret_cast<const h2*>(reinterpret_cast<const _Float16*>(a.wt.u_svh[e]) + col);
    const h2 sud = *reinterpret_cast<const h2*>(reinterpret_cast<const _Float16*>(a.wt.d_suh[e]) + col);
    const float L = a.limit;
    for (int rg2 = 0; rg2 < 4; ++rg2)
        for (int rb = 0; rb < 2; ++rb) {
            if (64 * rg2 + 32 * rb >= rn) continue;                 // uniform over the workgroup
            pf_stage_rows(acc, Cs, rg2, rb);
            __syncthreads();
            for (int rr = 0; rr < 4; ++rr) {
                const int rl = wv * 4 + rr;
                const int trow = 64 * rg2 + 32 * rb + rl;
                if (trow < rn) {
                    float g[2] = {Cs[rl * 256 + 2 * lane], Cs[rl * 256 + 2 * lane + 1]};
                    float u[2] = {Cs[rl * 256 + 128 + 2 * lane], Cs[rl * 256 + 128 + 2 * lane + 1]};
                    fwht128_w64(g[0], g[1], lane);
                    fwht128_w64(u[0], u[1], lane);
                    float b[2];
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        float gv = g[i] * HAD_R * (float)(i ? svg.y : svg.x);
                        float uv = u[i] * HAD_R * (float)(i ? svu.y : svu.x);
                        if (L != 0.0f) {
                            gv = fminf(gv, L);
                            uv = fminf(fmaxf(uv, -L), L);
                        }
                        const float act = sigmoid_dexp(gv) * gv * uv;
                        b[i] = (float)(_Float16)((_Float16)act * (i ? sud.y : sud.x));
                    }
                    fwht128_w64(b[0], b[1], lane);
                    *reinterpret_cast<h2*>(reinterpret_cast<_Float16*>(a.h2) + (size_t)(row0 + trow) * N + col) =
                        h2{(_Float16)(b[0] * HAD_R), (_Float16)(b[1] * HAD_R)};
                }
            }
            __syncthreads();
        }
}

// ------------------------------------------------------------------------------------------------ down

__global__ __launch_bounds__(PF_THREADS, 1) void pf_down_kernel(PrefillArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    int s, cb;
    pf_tile_of(blockIdx.x, a.K >> 8, s, cb);
    if (s >= a.nseg[0]) return;
    const int e = a.seg_expert[s], row0 = a.seg_row0[s], rn = a.seg_rows[s];
    const int K = a.K, N = a.N;
    PfTile t;
    t.a_rows = a.h2 + (size_t)row0 * N;
    t.rn = rn;
    t.kdim = N;
    t.btr[0] = t.btr[1] = reinterpret_cast<const uint32_t*>(a.wt.d_tr[e]);
    t.btiles_n = K >> 4;
    t.bcol0[0] = cb * 16;
    t.bcol0[1] = cb * 16 + 8;
    f16v acc[2][4];
    pf_gemm(t, smem, acc);

    float* Cs = reinterpret_cast<float*>(smem);
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const _Float16* svd = reinterpret_cast<const _Float16*>(a.wt.d_svh[e]) + cb * 256;
    const h2 sv0 = *reinterpret_cast<const h2*>(svd + 2 * lane);
    const h2 sv1 = *reinterpret_cast<const h2*>(svd + 128 + 2 * lane);
    for (int rg2 = 0; rg2 < 4; ++rg2)
        for (int rb = 0; rb < 2; ++rb) {
            if (64 * rg2 + 32 * rb >= rn) continue;
            pf_stage_rows(acc, Cs, rg2, rb);
            __syncthreads();
            for (int rr = 0; rr < 4; ++rr) {
                const int rl = wv * 4 + rr;
                const int trow = 64 * rg2 + 32 * rb + rl;
                if (trow < rn) {
                    const int row = row0 + trow;
                    const float w = (float)u16_as_h(a.w16[row]);
                    float* o = a.contrib + (size_t)row * K + cb * 256 + 2 * lane;
#pragma unroll
                    for (int hf = 0; hf < 2; ++hf) {
                        float v0 = Cs[rl * 256 + hf * 128 + 2 * lane], v1 = Cs[rl * 256 + hf * 128 + 2 * lane + 1];
                        fwht128_w64(v0, v1, lane);
                        const h2 sv = hf ? sv1 : sv0;
                        v0 = v0 * HAD_R * (float)sv.x * w;
                        v1 = v1 * HAD_R * (float)sv.y * w;
                        *reinterpret_cast<float2*>(o + hf * 128) = make_float2(v0, v1);
                    }
                }
            }
            __syncthreads();
        }
}

// ------------------------------------------------------------------------------------------------ combine

// grid (T, K/256), 128 threads x 2 columns: out[t] = sum over the token's slots k (in order) of the valid pairs'
// contributions, in the output dtype (deterministic: no atomics).
__global__ __launch_bounds__(128) void pf_combine_kernel(PrefillArgs a) {
    const int t = blockIdx.x;
    const int col = blockIdx.y * 256 + 2 * threadIdx.x;
    float s0 = 0.f, s1 = 0.f;
    for (int k = 0; k < a.topk; ++k) {
        const int pos = a.inv[t * a.topk + k];
        if (a.pe[pos] < 0) continue;
        const float2 c = *reinterpret_cast<const float2*>(a.contrib + (size_t)pos * a.K + col);
        s0 += c.x;
        s1 += c.y;
    }
    const size_t o = (size_t)t * a.out_stride + col;
    if (a.odt == DT_F32) {
        *reinterpret_cast<float2*>(reinterpret_cast<float*>(a.out) + o) = make_float2(s0, s1);
    } else if (a.odt == DT_BF16) {
        const uint32_t v = (uint32_t)f32_to_bf16(s0) | ((uint32_t)f32_to_bf16(s1) << 16);
        *reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(a.out) + o) = v;
    } else {
        *reinterpret_cast<h2*>(reinterpret_cast<uint16_t*>(a.out) + o) = h2{(_Float16)s0, (_Float16)s1};
    }
}

// ------------------------------------------------------------------------------------------------ launchers

static bool g_pf_attr = false;

int prefill_setup() {
    if (g_pf_attr) return 0;
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(pf_gateup_kernel),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)PF_LDS) != hipSuccess)
        return -1;
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(pf_down_kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)PF_LDS) != hipSuccess)
        return -1;
    g_pf_attr = true;
    return 0;
}

int launch_prefill(const PrefillArgs& a, hipStream_t st, int kernels) {
    if (prefill_setup()) return -1;
    if (kernels & 1) hipLaunchKernelGGL(pf_gather_kernel, dim3(4096), dim3(256), 0, st, a);
    const int sg = (a.S_cap + 7) / 8;                               // segment groups of 8 (one per XCD)
    if (kernels & 2)
        hipLaunchKernelGGL(pf_gateup_kernel, dim3(8 * (a.N / 128) * sg), dim3(PF_THREADS), PF_LDS, st, a);
    if (kernels & 4)
        hipLaunchKernelGGL(pf_down_kernel, dim3(8 * (a.K / 256) * sg), dim3(PF_THREADS), PF_LDS, st, a);
    if (kernels & 8) hipLaunchKernelGGL(pf_combine_kernel, dim3(a.T, a.K / 256), dim3(128), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace mi355moe
