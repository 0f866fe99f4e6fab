// Block-scaled e4m3 routed experts on gfx950's matrix cores: vLLM's fp8 w8a8 block-quantised MoE layout
// (w13 [n][2N][K] and w2 [n][K][N] e4m3 with one fp32 scale per 128x128 block) with per-token dynamic e4m3
// activations -- the e4m3 expert variant of the routed-MoE layer.
//
// Numerics (the reference's e4m3 contract, code/fork/kernels/moe_e4m3.cu:1-25 and :152-176,
// code/fork/overlay/glm53_moe_e4m3.py:648-674, with block-scaled weights in place of the trellis decode):
//   quant    per row: s = amax(|v|) / 448 (1 if 0), q = e4m3_rn(clamp(v / s, -448, 448))   (IEEE divisions)
//   gate/up  acc = sum over 128-k blocks b of (sum_{k in b} q_x[k] * W8[n][k]) * ws[n/128][b]  (exact products,
//            fp32 sums); g = acc * s_x, u likewise; a16 = fp16(silu(min(g, L)) * clamp(u, -L, L)) (iff L != 0),
//            silu(v) = v / (1 + (float)exp(-(double)v))
//   down     q_a, s_a = quant(a16 row); y = (same GEMM with the down scales) * s_a; contribution w * y per pair;
//            out[token] = the token's contributions summed in slot order (fp32), then the output dtype
//
// Work decomposition: a workgroup (4 waves) owns one 64-row segment of one expert and 64 output columns of gate and
// up (wave w: 32-row tile w / 2, columns 32 (w % 2) .. + 31 of both, so the SwiGLU is local to the lane; two
// workgroups per CU, which keeps more weight bytes in flight) or 128 output columns of down (wave w owns 32 of them
// for both 32-row tiles).
// Per 128-k block the workgroup stages its weight rows and activation rows in LDS with asynchronous
// global-to-LDS loads (three stages, two blocks in flight), each wave instruction reading whole 128-byte lines;
// lane half h = lane/32 then takes k 64h..64h+63 of its row from LDS. The e4m3 values are converted to fp16
// (exact: every e4m3 value is an fp16) and the block sum formed by eight v_mfma_f32_32x32x16_f16, each taking the
// same 8 of the lane's 64 k for both operands: every product is exact and the sums are fp32. (gfx950's fp8 MFMA,
// v_mfma_scale_f32_32x32x64_f8f6f4, aligns each group of 8 products to the group's largest and keeps ~12 bits,
// which left 0.9 % of the T=64 outputs of a 4096 x 1024 layer outside rtol 2e-2 / atol 1e-3 of the float64 layer;
// the fp16 form is ~12 % slower per layer and within 1e-7 of the fp32 sums.) The block sum is scaled by its
// weight scale in fp32 before it joins the accumulator.
#include "common.cuh"
#include "mi355moe_internal.h"

namespace mi355moe {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr float E4M3_MAX = 448.0f;

__device__ __forceinline__ float load_act(const void* x, int xdt, size_t i) {
    if (xdt == DT_F32) return reinterpret_cast<const float*>(x)[i];
    if (xdt == DT_BF16) return bf16_to_f32(reinterpret_cast<const uint16_t*>(x)[i]);
    return (float)u16_as_h(reinterpret_cast<const uint16_t*>(x)[i]);
}

// e4m3 codes (little-endian bytes) of four values already divided by their row scale: clamp to +-448, then
// round to nearest even (gfx950's fp8 conversion is OCP E4M3FN)
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
    a = __builtin_amdgcn_fmed3f(a, -E4M3_MAX, E4M3_MAX);
    b = __builtin_amdgcn_fmed3f(b, -E4M3_MAX, E4M3_MAX);
    c = __builtin_amdgcn_fmed3f(c, -E4M3_MAX, E4M3_MAX);
    d = __builtin_amdgcn_fmed3f(d, -E4M3_MAX, E4M3_MAX);
    int v = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    v = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, v, true);
    return (uint32_t)v;
}

// grid rows, 256 threads: q[r] = e4m3(clamp(x[r] / s[r])), s[r] = amax(|x[r]|) / 448 (1 if 0). K % 4 == 0.
__global__ __launch_bounds__(256) void quant_rows_kernel(const void* __restrict__ x, int xdt, int64_t stride, int K,
                                                         uint8_t* __restrict__ q, float* __restrict__ s) {
    __shared__ float red[4];
    const int r = blockIdx.x, tid = threadIdx.x;
    const size_t base = (size_t)r * stride;
    float m = 0.f;
    for (int c = tid * 4; c < K; c += 1024)
#pragma unroll
        for (int i = 0; i < 4; ++i) m = fmaxf(m, fabsf(load_act(x, xdt, base + c + i)));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float sc = __fdiv_rn(m, E4M3_MAX);
    sc = sc > 0.f ? sc : 1.f;
    if (tid == 0) s[r] = sc;
    for (int c = tid * 4; c < K; c += 1024) {
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = __fdiv_rn(load_act(x, xdt, base + c + i), sc);
        *reinterpret_cast<uint32_t*>(q + (size_t)r * K + c) = e4m3x4(v[0], v[1], v[2], v[3]);
    }
}

// The same quantisation with one wave per row and the row held in registers (4 rows per 256-thread workgroup): one
// read of the row, a wave maximum, K / 64 divisions per lane. G = K / 256 groups of four values per lane (lane l
// takes k = 256 g + 4 l .. + 3, so every wave load and store is contiguous). Same values as quant_rows_kernel.
template <int G>
__global__ __launch_bounds__(256) void quant_rows_wave_kernel(const void* __restrict__ x, int xdt, int64_t stride,
                                                              int rows, int K, uint8_t* __restrict__ q,
                                                              float* __restrict__ s) {
    const int r = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * 4 + (threadIdx.x >> 6)));
    if (r >= rows) return;
    const int lane = threadIdx.x & 63;
    const size_t base = (size_t)r * stride;
    float v[G][4];
    float m = 0.f;
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const size_t i0 = base + 256 * g + 4 * lane;
        if (xdt == DT_F32) {
            const float4 f = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(x) + i0);
            v[g][0] = f.x, v[g][1] = f.y, v[g][2] = f.z, v[g][3] = f.w;
        } else {
            const uint2 h = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(x) + i0);
            const uint32_t hv[2] = {h.x, h.y};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint16_t b = (uint16_t)(hv[i >> 1] >> (16 * (i & 1)));
                v[g][i] = xdt == DT_BF16 ? bf16_to_f32(b) : (float)u16_as_h(b);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) m = fmaxf(m, fabsf(v[g][i]));
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    float sc = __fdiv_rn(m, E4M3_MAX);
    sc = sc > 0.f ? sc : 1.f;
    if (lane == 0) s[r] = sc;
#pragma unroll
    for (int g = 0; g < G; ++g)
        *reinterpret_cast<uint32_t*>(q + (size_t)r * K + 256 * g + 4 * lane) =
            e4m3x4(__fdiv_rn(v[g][0], sc), __fdiv_rn(v[g][1], sc), __fdiv_rn(v[g][2], sc), __fdiv_rn(v[g][3], sc));
}

// Staging of one 128-k block of a workgroup tile in LDS: row R of the tile holds its 128 bytes as eight 16-byte
// chunks, chunk g at slot g ^ swz(R). The swizzle is applied through the load addresses (global_load_lds writes
// lane l of a wave instruction to slot l % 8 of row l / 8), so every wave instruction reads eight whole 128-byte
// lines, and the fragment reads below (32 consecutive rows, one chunk each) are free of bank conflicts.
__device__ __forceinline__ int swz(int R) { return (R >> 1) & 7; }

// The 64 bytes of row R at k half h (chunks 4h..4h+3) as four 16-byte LDS reads.
__device__ __forceinline__ void frag64(const unsigned char* st, int R, int h, u32x4 (&v)[4]) {
    const unsigned char* row = st + R * 128;
    const int sw = swz(R);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = *reinterpret_cast<const u32x4*>(row + (((4 * h + i) ^ sw) << 4));
}

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
// 16 e4m3 (one 16-byte chunk) -> 16 fp16 (exact), as two fp16 MFMA operands of 8 values each (scale 2^0; op_sel
// picks the dword's high two bytes)
__device__ __forceinline__ void e4m3_to_h16(const u32x4& q, h8& lo, h8& hi) {
    const float one = 1.0f;
    uint32_t d[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        asm("v_cvt_scalef32_pk_f16_fp8 %0, %1, %2" : "=v"(d[2 * i]) : "v"(q[i]), "v"(one));
        asm("v_cvt_scalef32_pk_f16_fp8 %0, %1, %2 op_sel:[1,0,0]" : "=v"(d[2 * i + 1]) : "v"(q[i]), "v"(one));
    }
    lo = __builtin_bit_cast(h8, u32x4{d[0], d[1], d[2], d[3]});
    hi = __builtin_bit_cast(h8, u32x4{d[4], d[5], d[6], d[7]});
}
// The 128-k block sum of one 32x32 tile from fp16-converted fragments (lane: 64 values of its row / column, the
// same k order for both operands), times its block scale, added to acc: eight v_mfma_f32_32x32x16_f16.
__device__ __forceinline__ void block_acc16(const h8 (&xa)[8], const h8 (&wb)[8], float ws, f32x16& acc) {
    f32x16 p = {};
#pragma unroll
    for (int i = 0; i < 8; ++i) p = __builtin_amdgcn_mfma_f32_32x32x16_f16(xa[i], wb[i], p, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] += p[i] * ws;
}

// Accumulator layout of a 32x32 tile: lane l holds column l % 32, register r row 8 (r / 4) + 4 (l / 32) + r % 4.
__device__ __forceinline__ int tile_row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }


constexpr int FP8_MAX_KB = 128;           // 128-k blocks per row (hidden and intermediate <= 16384)
constexpr int GU_ROWS = 192;              // 64 gate + 64 up weight rows + 64 activation rows per stage
constexpr int GU_INST = GU_ROWS / 8 / 4;  // wave instructions per stage per wave (6)
constexpr int DN_ROWS = 192;              // 128 weight rows + 64 activation rows
constexpr int DN_INST = DN_ROWS / 8 / 4;  // 6

// grid (N/64, segments), 256 threads: the 64-row segment's gate and up outputs of 64 columns, SwiGLU -> a16.
// Three LDS stages of 24 KB (two workgroups per CU); the loads for block kb + 2 are issued while block kb is
// multiplied.
__global__ __launch_bounds__(256) void fp8_gateup_kernel(Fp8Args a) {
    __shared__ __align__(16) unsigned char st0[GU_ROWS * 128];
    __shared__ __align__(16) unsigned char st1[GU_ROWS * 128];
    __shared__ __align__(16) unsigned char st2[GU_ROWS * 128];
    __shared__ float scl[2 * FP8_MAX_KB];
    __shared__ float rsx[64];                                        // the segment rows' activation scales
    const int cb = blockIdx.x, s = blockIdx.y;
    if (s >= a.nseg[0]) return;
    const int e = a.seg_expert[s], row0 = a.seg_row0[s], rn = a.seg_rows[s];
    if (rn <= 0) return;                                             // (no rows: nothing to stage or store)
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int K = a.K, N = a.N;
    const int nkb = K >> 7;

    // thread i < 64: the token of segment row i (its activation scale goes to LDS at the first step)
    const int ti = threadIdx.x;
    const int tk = a.tok[row0 + min(ti & 63, rn - 1)];
    // this lane's source rows for its six stage instructions (swizzled chunk offset included); the token ids of the
    // activation rows (stage rows 128 ..) are all loaded before any is used (one memory latency, not one per row)
    const uint8_t* src[GU_INST];
    int rtok[GU_INST];
#pragma unroll
    for (int j = 0; j < GU_INST; ++j) {
        const int R = wv * (GU_INST * 8) + j * 8 + (lane >> 3);
        rtok[j] = a.tok[row0 + min(max(R - 128, 0), rn - 1)];
    }
#pragma unroll
    for (int j = 0; j < GU_INST; ++j) {
        const int R = wv * (GU_INST * 8) + j * 8 + (lane >> 3);
        const uint8_t* rowp;
        if (R < 64) rowp = a.w13 + ((size_t)e * 2 * N + cb * 64 + R) * K;
        else if (R < 128) rowp = a.w13 + ((size_t)e * 2 * N + N + cb * 64 + (R - 64)) * K;
        else rowp = a.qx + (size_t)rtok[j] * K;
        src[j] = rowp + (((lane & 7) ^ swz(R)) << 4);
    }
    const int ldsw = wv * (GU_INST * 8) * 128;                       // this wave's first stage row
    auto issue = [&](unsigned char* st, int kb) {
#pragma unroll
        for (int j = 0; j < GU_INST; ++j) {                           // weight rows (read once) non-temporal
            if (wv * (GU_INST * 8) + j * 8 < 128) dma16_nt(src[j] + (size_t)kb * 128, st + ldsw + j * 1024);
            else dma16(src[j] + (size_t)kb * 128, st + ldsw + j * 1024);
        }
    };

    // the block scales of this column block (gate then up; thread i < 2 nkb <= 256) and the rows' activation scales
    // (thread i < 64) are loaded before the first staged loads and written to LDS at the first step: loads return in
    // issue order, so the first step's wait covers them, and the loop reads no global memory of its own
    // (unconditional loads at clamped indices: a conditional one would be waited for where its value is selected)
    const int tsc = min(ti, 2 * nkb - 1);
    const float scv = a.w13s[((size_t)e * (2 * N / 128) + (tsc < nkb ? 0 : N / 128) + cb / 2) * nkb +
                             (tsc < nkb ? tsc : tsc - nkb)];
    const float sxv = a.sx[tk];
    const int h = lane >> 5, c = lane & 31;
    const int rt = wv >> 1, ct = wv & 1;
    f32x16 g0 = {}, u0 = {};
    auto compute = [&](const unsigned char* st, int kb) {
        u32x4 wg[4], wu[4], x0[4];
        frag64(st, ct * 32 + c, h, wg);
        frag64(st, 64 + ct * 32 + c, h, wu);
        frag64(st, 128 + rt * 32 + c, h, x0);
        const float fg = scl[kb], fu = scl[nkb + kb];
        h8 xa[8], ga[8], ua[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            e4m3_to_h16(x0[i], xa[2 * i], xa[2 * i + 1]);
            e4m3_to_h16(wg[i], ga[2 * i], ga[2 * i + 1]);
            e4m3_to_h16(wu[i], ua[2 * i], ua[2 * i + 1]);
        }
        block_acc16(xa, ga, fg, g0);
        block_acc16(xa, ua, fu, u0);
    };
    // one pipeline step on stage buffer `cur` (block kb): wait for it, barrier, refill `nxt` (the buffer read in
    // the previous step) with block kb + 2, multiply
    auto step = [&](unsigned char* cur, unsigned char* nxt, int kb) {
        if (kb + 1 < nkb) WAIT_VM(GU_INST);
        else WAIT_VM(0);
        if (kb == 0) {                                               // (uniform) the scales, published by the barrier
            if (ti < 2 * nkb) scl[ti] = scv;
            if (ti < 64) rsx[ti] = sxv;
        }
        LDS_BARRIER();
        if (kb + 2 < nkb) issue(nxt, kb + 2);
        compute(cur, kb);
    };
    issue(st0, 0);
    if (nkb > 1) issue(st1, 1);
    for (int kb = 0; kb < nkb; kb += 3) {
        step(st0, st2, kb);
        if (kb + 1 < nkb) step(st1, st0, kb + 1);
        if (kb + 2 < nkb) step(st2, st1, kb + 2);
    }

    // epilogue: every row computed (rows past rn repeat row rn - 1, not stored), so the 16 rows' work is one block of
    // independent operations; the row scales come from LDS
    // Lanes c and c ^ 1 then trade one fp16 of each register pair r, r + 1 (DPP lane ^ 1): the even lane stores
    // columns (c, c + 1) of row(r), the odd lane those of row(r + 1), 4 bytes each.
    const float L = a.limit;
    const bool odd = c & 1;
    const int col = cb * 64 + ct * 32 + (c & ~1);
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
        uint32_t hv[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const float sxv = rsx[min(32 * rt + tile_row(r + i, lane), rn - 1)];
            float gv = g0[r + i] * sxv, uv = u0[r + i] * sxv;
            if (L != 0.0f) {
                gv = fminf(gv, L);
                uv = fminf(fmaxf(uv, -L), L);
            }
            const float act = __fdiv_rn(gv, 1.0f + (float)exp(-(double)gv)) * uv;
            hv[i] = h_as_u16((_Float16)act);
        }
        const uint32_t recv = (uint32_t)__builtin_amdgcn_mov_dpp((int)(odd ? hv[0] : hv[1]), 0xB1, 0xF, 0xF, true);
        const int row = 32 * rt + tile_row(r + (odd ? 1 : 0), lane);     // (r even: rows r, r + 1 are adjacent)
        const uint32_t pv = odd ? (recv | (hv[1] << 16)) : (hv[0] | (recv << 16));
        if (row < rn) *reinterpret_cast<uint32_t*>(a.a16 + (size_t)(row0 + row) * N + col) = pv;
    }
}

// grid (K/128, segments), 256 threads: the segment's down outputs of 128 columns, stored as each pair's weighted
// contribution (the combine adds a token's contributions in slot order).
// Three LDS stages of 24 KB.
__global__ __launch_bounds__(256) void fp8_down_kernel(Fp8Args a) {
    __shared__ __align__(16) unsigned char st0[DN_ROWS * 128];
    __shared__ __align__(16) unsigned char st1[DN_ROWS * 128];
    __shared__ __align__(16) unsigned char st2[DN_ROWS * 128];
    __shared__ float scl[FP8_MAX_KB];
    __shared__ float rsa[64], rw[64];                                // the segment rows' scales and router weights
    __shared__ int rok[64];                                          // and whether they hold a valid pair
    const int cb = blockIdx.x, s = blockIdx.y;
    if (s >= a.nseg[0]) return;
    const int e = a.seg_expert[s], row0 = a.seg_row0[s], rn = a.seg_rows[s];
    if (rn <= 0) return;                                             // (no rows: nothing to stage or store)
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int K = a.K, N = a.N;
    const int nkb = N >> 7;

    const uint8_t* src[DN_INST];
#pragma unroll
    for (int j = 0; j < DN_INST; ++j) {
        const int R = wv * (DN_INST * 8) + j * 8 + (lane >> 3);
        const uint8_t* rowp;
        if (R < 128) rowp = a.w2 + ((size_t)e * K + cb * 128 + R) * N;
        else rowp = a.qa + (size_t)(row0 + min(R - 128, rn - 1)) * N;
        src[j] = rowp + (((lane & 7) ^ swz(R)) << 4);
    }
    const int ldsw = wv * (DN_INST * 8) * 128;
    auto issue = [&](unsigned char* st, int kb) {
#pragma unroll
        for (int j = 0; j < DN_INST; ++j) {                           // weight rows (read once) non-temporal
            if (wv * (DN_INST * 8) + j * 8 < 128) dma16_nt(src[j] + (size_t)kb * 128, st + ldsw + j * 1024);
            else dma16(src[j] + (size_t)kb * 128, st + ldsw + j * 1024);
        }
    };
    // the block scales (thread i < nkb) and the rows' scales, router weights and validity (thread i < 64) are loaded
    // before the first staged loads and written to LDS at the first step (loads return in issue order)
    const int ti = threadIdx.x;
    // (unconditional loads at clamped indices: a conditional one would be waited for where its value is selected)
    const float scv = a.w2s[((size_t)e * (K / 128) + cb) * nkb + min(ti, nkb - 1)];
    const int rpos = row0 + min(ti & 63, rn - 1);
    const float sav = a.sa[rpos], rwv = a.w32[rpos];
    const int pev = a.pe[rpos];
    const int h = lane >> 5, c = lane & 31;
    f32x16 d0 = {}, d1 = {};
    auto compute = [&](const unsigned char* st, int kb) {
        u32x4 wd[4], x0[4], x1[4];
        frag64(st, wv * 32 + c, h, wd);
        frag64(st, 128 + c, h, x0);
        frag64(st, 160 + c, h, x1);
        const float fd = scl[kb];
        h8 wa[8], xa0[8], xa1[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            e4m3_to_h16(wd[i], wa[2 * i], wa[2 * i + 1]);
            e4m3_to_h16(x0[i], xa0[2 * i], xa0[2 * i + 1]);
            e4m3_to_h16(x1[i], xa1[2 * i], xa1[2 * i + 1]);
        }
        block_acc16(xa0, wa, fd, d0);
        block_acc16(xa1, wa, fd, d1);
    };
    auto step = [&](unsigned char* cur, unsigned char* nxt, int kb) {
        if (kb + 1 < nkb) WAIT_VM(DN_INST);
        else WAIT_VM(0);
        if (kb == 0) {                                               // (uniform) published by the barrier
            if (ti < nkb) scl[ti] = scv;
            if (ti < 64) {
                rsa[ti] = sav;
                rw[ti] = rwv;
                rok[ti] = ti < rn && pev >= 0;                      // (a pair whose token id was out of range: no row)
            }
        }
        LDS_BARRIER();
        if (kb + 2 < nkb) issue(nxt, kb + 2);
        compute(cur, kb);
    };
    issue(st0, 0);
    if (nkb > 1) issue(st1, 1);
    for (int kb = 0; kb < nkb; kb += 3) {
        step(st0, st2, kb);
        if (kb + 1 < nkb) step(st1, st0, kb + 1);
        if (kb + 2 < nkb) step(st2, st1, kb + 2);
    }

    // epilogue: every row computed from the LDS row factors, stored where the row holds a valid pair. Lanes c and
    // c ^ 1 (same rows, adjacent columns) trade one value of each register pair r, r + 1 (DPP lane ^ 1): the even
    // lane stores columns (c, c + 1) of row(r), the odd lane those of row(r + 1), 8 bytes each.
    const bool odd = c & 1;
    const int col = cb * 128 + wv * 32 + (c & ~1);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
            float v[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int rr = min(32 * t + tile_row(r + i, lane), 63);
                v[i] = rw[rr] * ((t ? d1[r + i] : d0[r + i]) * rsa[rr]);
            }
            const float send = odd ? v[0] : v[1];
            const float recv = __builtin_bit_cast(
                float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, send), 0xB1, 0xF, 0xF, true));
            const int row = 32 * t + tile_row(r + (odd ? 1 : 0), lane);   // (r even: rows r, r + 1 are adjacent)
            const float2 pv = odd ? make_float2(recv, v[1]) : make_float2(v[0], recv);
            if (rok[min(row, 63)]) *reinterpret_cast<float2*>(a.contrib + (size_t)(row0 + row) * K + col) = pv;
        }
    }
}

// grid (ceil(T/4), K/256), 256 threads: one wave per (token t, 256 columns), 4 columns per lane. out[t] = sum over
// the token's slots k (in order) of the valid pairs' contributions, converted to the output dtype (deterministic:
// no atomics).
__global__ __launch_bounds__(256) void fp8_combine_kernel(Fp8Args a) {
    const int t = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * 4 + (threadIdx.x >> 6)));
    if (t >= a.T) return;
    const int lane = threadIdx.x & 63;
    const int col = blockIdx.y * 256 + 4 * lane;
    float sum[4] = {0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < a.topk; k0 += 8) {
        // lanes 0..7 read slot k0 + lane's position and validity (broadcast by readlane); every slot's row is then
        // loaded before the first is added
        const int lk = k0 + (lane & 7);
        const int pl = a.inv[t * a.topk + min(lk, a.topk - 1)];
        const int okl = (int)(lk < a.topk && a.pe[pl] >= 0);
        float4 c[8];
        bool ok[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int pos = __builtin_amdgcn_readlane(pl, k);
            ok[k] = __builtin_amdgcn_readlane(okl, k) != 0;
            c[k] = *reinterpret_cast<const float4*>(a.contrib + (size_t)pos * a.K + col);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (ok[k]) {                                               // slot order
                sum[0] += c[k].x;
                sum[1] += c[k].y;
                sum[2] += c[k].z;
                sum[3] += c[k].w;
            }
    }
    const size_t o = (size_t)t * a.out_stride + col;
    if (a.odt == DT_F32) {
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(a.out) + o) = make_float4(sum[0], sum[1], sum[2], sum[3]);
    } else if (a.odt == DT_BF16) {
        *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(a.out) + o) =
            make_uint2(pack_bf16x2(sum[0], sum[1]), pack_bf16x2(sum[2], sum[3]));
    } else {
        h2* op = reinterpret_cast<h2*>(reinterpret_cast<uint16_t*>(a.out) + o);
        op[0] = h2{(_Float16)sum[0], (_Float16)sum[1]};
        op[1] = h2{(_Float16)sum[2], (_Float16)sum[3]};
    }
}

// ------------------------------------------------------------------------------------------------ launchers

// Rows of K = 256, 512, 1024, 2048 or 4096 values (and a 16-byte aligned source for fp32, 8-byte otherwise) take
// the one-wave-per-row kernel; other shapes the one-workgroup-per-row kernel.
static void quant_rows(const void* x, int xdt, int64_t stride, int rows, int K, uint8_t* q, float* s, hipStream_t st) {
    if (rows <= 0) return;
    const int align = xdt == DT_F32 ? 16 : 8;
    const bool wave = (reinterpret_cast<uintptr_t>(x) % align) == 0 && stride % 4 == 0;
    const dim3 grid((rows + 3) / 4);
    if (wave && K == 4096) hipLaunchKernelGGL(quant_rows_wave_kernel<16>, grid, dim3(256), 0, st, x, xdt, stride, rows, K, q, s);
    else if (wave && K == 2048) hipLaunchKernelGGL(quant_rows_wave_kernel<8>, grid, dim3(256), 0, st, x, xdt, stride, rows, K, q, s);
    else if (wave && K == 1024) hipLaunchKernelGGL(quant_rows_wave_kernel<4>, grid, dim3(256), 0, st, x, xdt, stride, rows, K, q, s);
    else if (wave && K == 512) hipLaunchKernelGGL(quant_rows_wave_kernel<2>, grid, dim3(256), 0, st, x, xdt, stride, rows, K, q, s);
    else if (wave && K == 256) hipLaunchKernelGGL(quant_rows_wave_kernel<1>, grid, dim3(256), 0, st, x, xdt, stride, rows, K, q, s);
    else hipLaunchKernelGGL(quant_rows_kernel, dim3(rows), dim3(256), 0, st, x, xdt, stride, K, q, s);
}

int launch_quant_rows(const void* x, int xdt, int64_t stride, int rows, int K, uint8_t* q, float* s, hipStream_t st) {
    quant_rows(x, xdt, stride, rows, K, q, s, st);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_fp8(const Fp8Args& a, hipStream_t st, int kernels) {
    if (kernels & 1)
        quant_rows(a.x, a.xdt, a.x_stride, a.T, a.K, a.qx, a.sx, st);
    if (kernels & 2) hipLaunchKernelGGL(fp8_gateup_kernel, dim3(a.N / 64, a.S_cap), dim3(256), 0, st, a);
    if (kernels & 4) {
        quant_rows(a.a16, DT_F16, a.N, a.P, a.N, a.qa, a.sa, st);
        hipLaunchKernelGGL(fp8_down_kernel, dim3(a.K / 128, a.S_cap), dim3(256), 0, st, a);
    }
    if (kernels & 8) hipLaunchKernelGGL(fp8_combine_kernel, dim3((a.T + 3) / 4, a.K / 256), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace mi355moe
