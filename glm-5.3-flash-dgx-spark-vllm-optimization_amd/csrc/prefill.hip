// Prefill-path kernels (many rows per expert, the E3 grouped tier): gather + input rotation, the gate/up grouped
// GEMM and the down grouped GEMM on fp16 MFMA (v_mfma_f32_32x32x16_f16) with the EXL3 trellis decoded in registers.
//
// Tiles: a workgroup of 4 waves (one per SIMD) owns a 256-row segment of one expert (rows sorted by expert) and one
// column block; each wave multiplies all 256 rows by its own 64 columns:
//   gate/up: 128 columns of gate (waves 0, 1) and the same 128 of up (waves 2, 3);
//   down:    256 output columns.
// The A rows are staged in LDS (shared by the 4 waves); each wave decodes its own trellis words straight into MFMA
// operands, so every weight value is decoded once per tile and never goes through LDS. Calls with few rows per
// expert run the same GEMM on 128- or 64-row parts of the segments instead (the mid- and small-tile kernels: two
// workgroups per CU, see pf_tiles).
// Numerics (oracle/csrc/oracle.c mode 1 = the E3 kernels, code/fork/docs/ref/mia_exl3-fat-kernel/exl3_fat_moe.cu):
//   gather   h13 = fp16(H(fp16(x * suh_g)) * r)                                         (exl3_fat_moe.cu:95-126)
//   gate/up  g = (H(acc_g) * r) * svh_g, u likewise; iff L != 0: g = min(g, L), u = clamp(u, -L, L);
//            a = sigmoid(g) * g * u; h2 = fp16(H(fp16(fp16(a) * suh_d)) * r)  (:340-378; the reference's sigmoid is
//            1 / (1 + (float)exp(-(double)g)), here an fp32 one within a few ulp of it)
//   down     contribution ((H(acc_d) * r) * svh_d) * w16 per pair                       (:443-457); out[token] =
//            the token's contributions summed in slot order (fp32), then the output dtype. The down kernel stores the
//            raw accumulators acc_d; the combine applies H, r, svh_d and w16 before summing.
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "common.cuh"
#include "mi355moe_internal.h"

namespace mi355moe {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));

constexpr int PF_TM = PREFILL_TM;   // rows per tile (segment height)
constexpr int PF_THREADS = 256;     // 4 waves, one per SIMD: each owns 64 columns of the tile for all 256 rows
constexpr int PF_KT = 4;            // 16-k trellis tiles per step (one wait + barrier per step)
constexpr int PF_NS = 4;            // staged steps in flight (A rows and raw trellis words)
constexpr int PF_RB = 32 * PF_KT;               // bytes of one A row in a stage (fp16, k permuted as stored)
constexpr int PF_ASB = PF_TM * PF_RB;           // one A stage: 256 rows x 16 PF_KT k
constexpr int PF_WWB = 512 * PF_KT;             // one wave's raw words of a step: PF_KT k tiles x 4 column tiles x 128 B
constexpr int PF_WSB = 4 * PF_WWB;              // one raw-word stage (4 waves)
constexpr size_t PF_LDS = (size_t)PF_NS * (PF_ASB + PF_WSB);   // 163,840 bytes (the whole LDS)
constexpr int PF_TMS = 64;                      // rows per tile of the small-tile kernels (two per CU)
constexpr size_t PF_LDS_S = (size_t)PF_NS * (PF_TMS * PF_RB + PF_WSB);   // 65,536 bytes
constexpr int PF_TMM = 128;                     // rows per tile of the mid-tile kernels (two per CU)
constexpr int PF_NSM = 3;                       // their staged steps
constexpr size_t PF_LDS_M = (size_t)PF_NSM * (PF_TMM * PF_RB + PF_WSB);  // 73,728 bytes
// Tile kinds of the grouped GEMMs: the rows of a segment (at most 256) taken whole, in 64-row quarters or in
// 128-row halves.
enum { PF_LARGE = 0, PF_SMALL = 1, PF_MID = 2 };
__host__ __device__ constexpr int pf_sub_rows(int kind) { return kind == PF_SMALL ? PF_TMS : kind == PF_MID ? PF_TMM : PF_TM; }
constexpr int PF_CLD = 260;                     // epilogue staging row stride (floats): [32][PF_CLD] fp32
// Row blocks (32 rows each) the gate/up epilogue stages at once: as many as the kernel's LDS holds.
__host__ __device__ constexpr int pf_epi_blocks(int kind) {
    return (int)((kind == PF_SMALL ? PF_LDS_S : kind == PF_MID ? PF_LDS_M : PF_LDS) / (32 * PF_CLD * 4));
}

// Rotated activations (h13, h2) are stored with k permuted inside every group of 16: storage pair p (halves 2p,
// 2p+1) holds k pair j with p = 2 (j % 4) + j / 4, i.e. storage order k = 0,1,8,9, 2,3,10,11, 4,5,12,13, 6,7,14,15.
// That is the k order in which one lane decodes two consecutive trellis words of a column, so the decoded weights
// go straight into MFMA operands (8 consecutive k slots per lane) and the activations match them slot for slot.
__device__ __forceinline__ int pf_kperm_pair(int j) { return 2 * (j & 3) + (j >> 2); }

// Store a lane's four packed pairs (k pairs 4h .. 4h + 3 of 16-group g, lane c = 2g + h) at their permuted positions
// with one 16-byte store: the lanes c, c ^ 1 of a group own its 32 bytes interleaved (storage pair 2m + h = the lane's
// pair m), so they swap two pairs (DPP lane ^ 1) and lane h then writes storage pairs 4h .. 4h + 3 contiguously.
// grp: the 16-group's first element.
__device__ __forceinline__ u32x4 pf_group_vec(const uint32_t (&wm)[4], int c) {
    const bool hi = c & 1;
    const uint32_t s0 = hi ? wm[0] : wm[2], s1 = hi ? wm[1] : wm[3];
    const uint32_t r0 = (uint32_t)__builtin_amdgcn_mov_dpp((int)s0, 0xB1, 0xF, 0xF, true);   // lane ^ 1
    const uint32_t r1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)s1, 0xB1, 0xF, 0xF, true);
    return hi ? u32x4{r0, wm[2], r1, wm[3]} : u32x4{wm[0], r0, wm[1], r1};
}
__device__ __forceinline__ void pf_store_group(_Float16* grp, const uint32_t (&wm)[4], int c) {
    *reinterpret_cast<u32x4*>(grp + 8 * (c & 1)) = pf_group_vec(wm, c);
}
// The same as one device-coherent store, for rows that workgroups on other XCDs read in the same launch: r over the
// row block, grp_off the 16-group's byte offset in it.
__device__ __forceinline__ void pf_store_group_coh(__amdgpu_buffer_rsrc_t r, int grp_off, const uint32_t (&wm)[4],
                                                   int c) {
    st_coh16(r, grp_off + 16 * (c & 1), pf_group_vec(wm, c));
}
__device__ __forceinline__ float4 f4_of(u32x4 v) {
    const f32x4 f = __builtin_bit_cast(f32x4, v);
    return make_float4(f[0], f[1], f[2], f[3]);
}

// The same placement for one byte per element (e4m3 codes): q[m] holds the lane's pair m as two codes in its low 16
// bits; lane h of the pair of lanes writes storage pairs 4h .. 4h + 3 as 8 contiguous bytes. grp: the 16-group's
// first byte.
__device__ __forceinline__ void pf_store_group8(uint8_t* grp, const uint32_t (&q)[4], int c) {
    const bool hi = c & 1;
    const uint32_t s = hi ? (q[0] | (q[1] << 16)) : (q[2] | (q[3] << 16));
    const uint32_t r = (uint32_t)__builtin_amdgcn_mov_dpp((int)s, 0xB1, 0xF, 0xF, true);   // lane ^ 1
    const uint2 v = hi ? make_uint2((r & 0xFFFFu) | (q[2] << 16), (r >> 16) | (q[3] << 16))
                       : make_uint2(q[0] | (r << 16), q[1] | (r & 0xFFFF0000u));
    *reinterpret_cast<uint2*>(grp + 8 * (c & 1)) = v;
}

// ------------------------------------------------------------------------------------------------ gather

// Work item i of a gather: the row it writes, the token it reads and the expert whose suh it applies; false when the
// item is skipped (see PrefillArgs: sorted positions with pe/tok, caller row tables with tok64, or routed pairs).
__device__ __forceinline__ bool pf_gather_item(const PrefillArgs& a, int i, int& pos, int& tok, int& e) {
    if (a.tok_rows) {                                                 // one row per token, the layer's one suh
        pos = tok = i;
        e = 0;
        return true;
    }
    if (a.pair_pos) {
        e = a.pair_local[i];
        if (e < 0 || e >= a.n) return false;
        pos = a.pair_pos[i];
        if (pos < 0 || pos >= a.P) return false;                      // (caller-built tables)
        tok = i / a.topk;
        return true;
    }
    e = a.pe[i];
    if (e < 0 || e >= a.n) return false;
    pos = i;
    if (a.tok64) {
        const int64_t t = a.tok64[i];
        if (t < 0 || t >= a.T) return false;                         // (caller-built tables)
        tok = (int)t;
    } else {
        tok = a.tok ? a.tok[i] : i;                                   // no token table: row i reads x row i
    }
    return true;
}
// Number of work items of a gather (a device row count caps the caller's row tables).
__device__ __forceinline__ int pf_gather_items(const PrefillArgs& a) {
    if (a.tok_rows) return a.T;
    return a.nrows ? min(a.P, __builtin_amdgcn_readfirstlane(a.nrows[0])) : a.P;
}

// h13[pos] = rotated x[tok[pos]] with expert pe[pos]'s gate suh, for every row with pe >= 0 (tok_rows: h13[t] =
// rotated x[t] with the suh every expert shares, for every token t). One wave per row
// (grid-stride): a pass rotates four 128-blocks at once (16 lanes per block, lane c holding elements 8c .. 8c + 7,
// DPP Hadamard); the loads of all passes of the row are issued before the first rotation.
constexpr int PF_GATHER_PASSES = 8;                 // passes of 4 blocks in flight (K up to 4096 in one round)
__global__ __launch_bounds__(256) void pf_gather_kernel(PrefillArgs a) {
    if (a.sched && blockIdx.x == 0)                                   // the one-launch schedule's control words
        for (int i = threadIdx.x; i < PF_SCHED_WORDS(a.S_cap); i += 256) a.sched[i] = 0;
    const int lane = threadIdx.x & 63;
    const int c = lane & 15, q = lane >> 4;
    const int nb = a.K >> 7;
    const bool vec = ((reinterpret_cast<uintptr_t>(a.x) | ((uintptr_t)a.x_stride * 2)) & 15) == 0;
    const int wave = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * 4 + (threadIdx.x >> 6)));
    const int items = pf_gather_items(a);
    for (int it = wave; it < items; it += gridDim.x * 4) {
        int pos, tk, e;
        if (!pf_gather_item(a, it, pos, tk, e)) continue;             // uniform: one row per wave
        const uint16_t* xr = reinterpret_cast<const uint16_t*>(a.x) + (size_t)tk * a.x_stride + 8 * c;
        const uint16_t* sr = reinterpret_cast<const uint16_t*>(a.wt.g_suh[e]) + 8 * c;
        _Float16* dst0 = reinterpret_cast<_Float16*>(a.h13) + (size_t)pos * a.K + 16 * (c >> 1);
        for (int b0 = 0; b0 < nb; b0 += 4 * PF_GATHER_PASSES) {
            u32x4 xv[PF_GATHER_PASSES], sv[PF_GATHER_PASSES];
#pragma unroll
            for (int j = 0; j < PF_GATHER_PASSES; ++j) {
                const int blk = min(b0 + 4 * j + q, nb - 1);
                const uint16_t* xp = xr + blk * 128;
                if (vec) {
                    xv[j] = *reinterpret_cast<const u32x4*>(xp);
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) xv[j][i] = *reinterpret_cast<const uint32_t*>(xp + 2 * i);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) sv[j][i] = *reinterpret_cast<const uint32_t*>(sr + blk * 128 + 2 * i);
            }
#pragma unroll
            for (int j = 0; j < PF_GATHER_PASSES; ++j) {
                const int blk = b0 + 4 * j + q;
                if (b0 + 4 * j >= nb) break;                          // uniform
                float p[8];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t v = xv[j][i];
                    _Float16 h0, h1;
                    if (a.xdt == DT_BF16) {
                        h0 = (_Float16)__builtin_bit_cast(float, v << 16);
                        h1 = (_Float16)__builtin_bit_cast(float, v & 0xFFFF0000u);
                    } else {
                        h0 = u16_as_h(v & 0xFFFFu);
                        h1 = u16_as_h(v >> 16);
                    }
                    const uint32_t sw = sv[j][i];
                    p[2 * i] = (float)(_Float16)(h0 * u16_as_h(sw & 0xFFFFu));
                    p[2 * i + 1] = (float)(_Float16)(h1 * u16_as_h(sw >> 16));
                }
                fwht128_x16s(p, lane);
                const float hr = HAD_R * fwht_sign(lane);
                uint32_t wm[4];
#pragma unroll
                for (int m = 0; m < 4; ++m)
                    wm[m] = __builtin_bit_cast(uint32_t, h2{(_Float16)(p[2 * m] * hr), (_Float16)(p[2 * m + 1] * hr)});
                if (blk < nb) pf_store_group(dst0 + blk * 128, wm, c);
            }
        }
    }
}

// ------------------------------------------------------------------------------------------------ e4m3 helpers

// Two fp16 values (|v| <= 448) rounded to their nearest e4m3 values (ties to even, e4m3 subnormals included), returned
// as the fp16 pair of those values (every e4m3 value is an fp16): gfx950's scaled conversions with scale 1.
__device__ __forceinline__ uint32_t e4m3_round_h2(uint32_t d) {
    const float one = 1.0f;
    uint32_t f8, r;
    asm("v_cvt_scalef32_pk_fp8_f16 %0, %1, %2" : "=v"(f8) : "v"(d), "v"(one));
    asm("v_cvt_scalef32_pk_f16_fp8 %0, %1, %2" : "=v"(r) : "v"(f8), "v"(one));
    return r;
}
// Two fp32 values already divided by their row scale -> the codes of e4m3(clamp(v, -448, 448)) in the low 16 bits
// (round to nearest even, the reference's quantiser); e4m3_h2 widens two codes to the fp16 pair of their values.
__device__ __forceinline__ uint32_t e4m3_quant_f8(float a, float b) {
    a = __builtin_amdgcn_fmed3f(a, -448.0f, 448.0f);
    b = __builtin_amdgcn_fmed3f(b, -448.0f, 448.0f);
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xFFFFu;
}
__device__ __forceinline__ uint32_t e4m3_h2(uint32_t f8) {
    const float one = 1.0f;
    uint32_t r;
    asm("v_cvt_scalef32_pk_f16_fp8 %0, %1, %2" : "=v"(r) : "v"(f8), "v"(one));
    return r;
}
__device__ __forceinline__ uint32_t e4m3_quant_h2(float a, float b) { return e4m3_h2(e4m3_quant_f8(a, b)); }
// Row scale of the e4m3 activations: amax / 448 (IEEE division), 1 for an all-zero row.
__device__ __forceinline__ float e4m3_row_scale(float amax) {
    const float sc = __fdiv_rn(amax, 448.0f);
    return sc > 0.0f ? sc : 1.0f;
}

// The e4m3 variant's gather (code/fork/kernels/moe_e4m3.cu:245-310, gather2; with tok_rows one row per token, its
// gather_tok; over rows with pe >= 0 and no token table, its actq :440-488 with x = the SwiGLU output and suh = the
// down suh): per row, v = H(x16 * suh) * r in fp32
// (x rounded to fp16 first, the product and the butterflies in fp32, r applied after the transform), s = amax|v| /
// 448, q = e4m3(clamp(v / s)) stored as the fp16 of each e4m3 value in h13's permuted order (a8out: as the e4m3 codes,
// one byte each, in that order), asc[pos] = s; the row's down-input maximum amaxd[pos] is zeroed for the gate/up
// epilogue. One wave per row; the whole row (K <= 4096) stays in registers between the amax and the quantization.
__global__ __launch_bounds__(256) void pf_gather8_kernel(PrefillArgs a) {
    if (a.sched && blockIdx.x == 0)                                   // the one-launch schedule's control words
        for (int i = threadIdx.x; i < PF_SCHED_WORDS(a.S_cap); i += 256) a.sched[i] = 0;
    const int lane = threadIdx.x & 63;
    const int c = lane & 15, q = lane >> 4;
    const int nb = a.K >> 7;
    const bool vec = ((reinterpret_cast<uintptr_t>(a.x) | ((uintptr_t)a.x_stride * 2)) & 15) == 0;
    const int wave = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * 4 + (threadIdx.x >> 6)));
    const int items = pf_gather_items(a);
    for (int it = wave; it < items; it += gridDim.x * 4) {
        int pos, tk, e;
        if (!pf_gather_item(a, it, pos, tk, e)) continue;             // uniform: one row per wave
        const uint16_t* xr = reinterpret_cast<const uint16_t*>(a.x) + (size_t)tk * a.x_stride + 8 * c;
        const uint16_t* sr = reinterpret_cast<const uint16_t*>(a.wt.g_suh[e]) + 8 * c;
        u32x4 xv[PF_GATHER_PASSES], sv[PF_GATHER_PASSES];
#pragma unroll
        for (int j = 0; j < PF_GATHER_PASSES; ++j) {
            const int blk = min(4 * j + q, nb - 1);
            const uint16_t* xp = xr + blk * 128;
            if (vec) {
                xv[j] = *reinterpret_cast<const u32x4*>(xp);
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) xv[j][i] = *reinterpret_cast<const uint32_t*>(xp + 2 * i);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) sv[j][i] = *reinterpret_cast<const uint32_t*>(sr + blk * 128 + 2 * i);
        }
        float v[PF_GATHER_PASSES][8];
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < PF_GATHER_PASSES; ++j) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t xw = xv[j][i], sw = sv[j][i];
                _Float16 h0, h1;
                if (a.xdt == DT_BF16) {
                    h0 = (_Float16)__builtin_bit_cast(float, xw << 16);
                    h1 = (_Float16)__builtin_bit_cast(float, xw & 0xFFFF0000u);
                } else {
                    h0 = u16_as_h(xw & 0xFFFFu);
                    h1 = u16_as_h(xw >> 16);
                }
                v[j][2 * i] = (float)h0 * (float)u16_as_h(sw & 0xFFFFu);
                v[j][2 * i + 1] = (float)h1 * (float)u16_as_h(sw >> 16);
            }
            fwht128_x16s(v[j], lane);
            const bool live = 4 * j + q < nb;
            const float hr = HAD_R * fwht_sign(lane);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                v[j][i] = v[j][i] * hr;
                if (live) m = fmaxf(m, fabsf(v[j][i]));
            }
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
        const float sc = e4m3_row_scale(m);
        _Float16* dst0 = reinterpret_cast<_Float16*>(a.h13) + (size_t)pos * a.K + 16 * (c >> 1);
        uint8_t* dst8 = a.a8out + (size_t)pos * a.K + 16 * (c >> 1);
#pragma unroll
        for (int j = 0; j < PF_GATHER_PASSES; ++j) {
            const int blk = 4 * j + q;
            if (blk < nb) {
                uint32_t wm[4];
#pragma unroll
                for (int mm = 0; mm < 4; ++mm)
                    wm[mm] = e4m3_quant_f8(__fdiv_rn(v[j][2 * mm], sc), __fdiv_rn(v[j][2 * mm + 1], sc));
                if (a.a8out) {                                       // the codes (the extension's byte layout)
                    pf_store_group8(dst8 + blk * 128, wm, c);
                } else {
#pragma unroll
                    for (int mm = 0; mm < 4; ++mm) wm[mm] = e4m3_h2(wm[mm]);
                    pf_store_group(dst0 + blk * 128, wm, c);
                }
            }
        }
        if (lane == 0) {
            a.asc[pos] = sc;
            if (a.amaxd && !a.tok_rows) a.amaxd[pos] = 0u;
        }
    }
    if (a.amaxd && a.tok_rows)                                       // rows, not tokens: zeroed by a grid-stride loop
        for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < a.P; i += gridDim.x * blockDim.x) a.amaxd[i] = 0u;
}

// The e4m3 variant's down-input quantization: per row, s = amaxd / 448 (the maximum over the whole row, gathered by
// the gate/up epilogues), h2 = the fp16 of e4m3(clamp(vd / s)) in the permuted order (a8dout: also the codes, one
// byte each, in that order), dsc[pos] = s. One wave per row, four 128-blocks per pass.
// One row of it, by one wave. COH: vd and amaxd were written in the same launch (possibly on other XCDs) and h2 is read
// there: device-coherent loads and stores.
template <bool COH>
__device__ __forceinline__ void pf_quantd_row(const PrefillArgs& a, int pos, int lane) {
    const int c = lane & 15, q = lane >> 4;
    // the row's expert, maximum and first values are loaded together (a row without an expert is read, not
    // written), so the row costs one memory latency instead of three
    const int pe = a.pe[pos];
    const float amax = __builtin_bit_cast(
        float, COH ? __hip_atomic_load(a.amaxd + pos, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : a.amaxd[pos]);
    const float* src = a.vd + (size_t)pos * a.N + 8 * c;
    const int nb = a.N >> 7;
    // pos is wave-uniform: the coherent accesses go through buffer resources over the row
    const __amdgpu_buffer_rsrc_t rv = coh_rsrc(a.vd + (size_t)pos * a.N);
    const __amdgpu_buffer_rsrc_t rh = coh_rsrc(reinterpret_cast<_Float16*>(a.h2) + (size_t)pos * a.N);
    auto ld4 = [&](int e) {                                   // the lane's floats e .. e + 3
        return COH ? f4_of(ld_coh16(rv, 4 * (8 * c + e))) : *reinterpret_cast<const float4*>(src + e);
    };
    float4 lo0 = {}, hi0 = {};
    if (q < nb) {
        lo0 = ld4(q * 128);
        hi0 = ld4(q * 128 + 4);
    }
    if (pe < 0) return;
    const float sc = e4m3_row_scale(amax);
    _Float16* dst0 = reinterpret_cast<_Float16*>(a.h2) + (size_t)pos * a.N + 16 * (c >> 1);
    uint8_t* dst8 = a.a8dout + (size_t)pos * a.N + 16 * (c >> 1);
    for (int blk = q; blk < nb; blk += 4) {
        const float4 lo = blk == q ? lo0 : ld4(blk * 128);
        const float4 hi = blk == q ? hi0 : ld4(blk * 128 + 4);
        const float w[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
        uint32_t f8[4], wm[4];
#pragma unroll
        for (int mm = 0; mm < 4; ++mm) {
            f8[mm] = e4m3_quant_f8(__fdiv_rn(w[2 * mm], sc), __fdiv_rn(w[2 * mm + 1], sc));
            wm[mm] = e4m3_h2(f8[mm]);
        }
        if (COH)
            pf_store_group_coh(rh, 2 * (16 * (c >> 1) + blk * 128), wm, c);
        else
            pf_store_group(dst0 + blk * 128, wm, c);
        if (a.a8dout) pf_store_group8(dst8 + blk * 128, f8, c);
    }
    if (lane == 0) a.dsc[pos] = sc;
}
// Rows pos0, pos0 + step, ... (R of them, below end) by one wave, device-coherent, with every row's maximum and values
// loaded before the first is quantised (one memory latency for the R rows; N <= 1024: two 128-blocks per lane).
template <int R>
__device__ __forceinline__ void pf_quantd_rows_coh(const PrefillArgs& a, int pos0, int step, int end, int lane) {
    const int c = lane & 15, q = lane >> 4;
    const int nb = a.N >> 7;
    int pos[R], pe[R];
    float amax[R];
    float4 v[R][4];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        pos[r] = min(pos0 + r * step, end - 1);
        pe[r] = pos0 + r * step < end ? a.pe[pos[r]] : -1;
        amax[r] = __builtin_bit_cast(float, __hip_atomic_load(a.amaxd + pos[r], __ATOMIC_RELAXED,
                                                              __HIP_MEMORY_SCOPE_AGENT));
        const __amdgpu_buffer_rsrc_t rv = coh_rsrc(a.vd + (size_t)pos[r] * a.N);   // (pos0, step: wave-uniform)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int blk = q + 4 * j;
            v[r][2 * j] = v[r][2 * j + 1] = float4{};
            if (blk < nb) {
                v[r][2 * j] = f4_of(ld_coh16(rv, 4 * (8 * c + blk * 128)));
                v[r][2 * j + 1] = f4_of(ld_coh16(rv, 4 * (8 * c + blk * 128 + 4)));
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (pe[r] < 0) continue;                                      // (uniform)
        const float sc = e4m3_row_scale(amax[r]);
        const __amdgpu_buffer_rsrc_t rh = coh_rsrc(reinterpret_cast<_Float16*>(a.h2) + (size_t)pos[r] * a.N);
        uint8_t* dst8 = a.a8dout + (size_t)pos[r] * a.N + 16 * (c >> 1);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int blk = q + 4 * j;
            if (blk >= nb) continue;
            const float w[8] = {v[r][2 * j].x, v[r][2 * j].y, v[r][2 * j].z, v[r][2 * j].w,
                                v[r][2 * j + 1].x, v[r][2 * j + 1].y, v[r][2 * j + 1].z, v[r][2 * j + 1].w};
            uint32_t f8[4], wm[4];
#pragma unroll
            for (int mm = 0; mm < 4; ++mm) {
                f8[mm] = e4m3_quant_f8(__fdiv_rn(w[2 * mm], sc), __fdiv_rn(w[2 * mm + 1], sc));
                wm[mm] = e4m3_h2(f8[mm]);
            }
            pf_store_group_coh(rh, 2 * (16 * (c >> 1) + blk * 128), wm, c);
            if (a.a8dout) pf_store_group8(dst8 + blk * 128, f8, c);
        }
        if (lane == 0) a.dsc[pos[r]] = sc;
    }
}
__global__ __launch_bounds__(256) void pf_quantd_kernel(PrefillArgs a) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * 4 + (threadIdx.x >> 6)));
    for (int pos = wave; pos < a.P; pos += gridDim.x * 4) pf_quantd_row<false>(a, pos, lane);
}

// ------------------------------------------------------------------------------------------------ GEMM core

// The tile GEMM of one wave: acc[rb][s] (32x32 blocks, rows 32 rb of the segment) over kdim, for the wave's 64
// columns = four trellis column tiles. MFMA column n of block s is column 16 (n / 8) + n % 8 + 8 s of the wave.
// A rows come from `a_rows` (row stride kdim, k permuted as stored), clamped to rn - 1.
struct PfTile {
    const uint16_t* a_rows;       // first row of the segment (a_tok: row 0 of the token-row buffer)
    const int* a_tok;             // nullptr, or the segment's rows' tokens: row r is a_rows[a_tok[r]]
    int rn, kdim;
    const uint32_t* btr;          // this wave's trellis matrix
    int btiles_n;                 // tiles per trellis row (the matrix's column tiles)
    int bcol0;                    // this wave's first column tile
};

// A stage row R: PF_RB bytes = 2 PF_KT 16-byte chunks (storage k 8g .. 8g + 7), chunk g at slot g ^ pf_swz(R): the
// fragment reads (16 consecutive rows per LDS pass, one chunk each) then touch every bank once.
__device__ __forceinline__ int pf_swz(int R) { return PF_RB == 64 ? (R >> 2) & 3 : (R >> 1) & 7; }

// Decoded B operands, one fp16 pair at a time. Lane (n = lane % 32, h = lane / 32) of a k tile reads words
// wp = 4c + 2h and wp + 1 of column tile t (c = n % 8, t = n / 8) and the predecessor word wp - 1 (mod 32):
// w[0] = word wp - 1, w[1] = word wp, w[2] = word wp + 1. Pair p (0..7) of the lane: word wp (p < 4) or wp + 1,
// states 2 (p % 4) and 2 (p % 4) + 1 of that word (decode_word's order); the operand of column 16t + c is pairs
// 0, 1, 4, 5 (k slots 8h .. 8h + 7) and that of column 16t + c + 8 is pairs 2, 3, 6, 7.
__device__ __forceinline__ void pf_load_words(const unsigned char* wk, int lane, uint32_t (&w)[3]) {
    const int n = lane & 31, wp = 4 * (n & 7) + 2 * (lane >> 5);
    const unsigned char* tile = wk + (n >> 3) * 128;
    const uint2 v = *reinterpret_cast<const uint2*>(tile + 4 * wp);
    w[0] = *reinterpret_cast<const uint32_t*>(tile + 4 * ((wp + 31) & 31));
    w[1] = v.x;
    w[2] = v.y;
}
// The pair's decode in two halves (software-pipelined across MFMA pairs by the GEMM loop): pf_pair_products =
// the two states times MCG_MUL, pf_pair_values = mask, flip and the fp16 sums.
struct PfPair {
    uint32_t x0, x1;
};
__device__ __forceinline__ PfPair pf_pair_products(const uint32_t (&w)[3], int p) {
    const uint32_t pw = w[p >> 2], x = w[(p >> 2) + 1];
    uint32_t s0, s1;
    switch (p & 3) {
        case 0: {
            const uint32_t D = __builtin_amdgcn_alignbit(pw, x, 20);
            s0 = __builtin_amdgcn_ubfe(D, 8, 16);
            s1 = __builtin_amdgcn_ubfe(D, 4, 16);
            break;
        }
        case 1:
            s0 = __builtin_amdgcn_alignbit(pw, x, 20) & 0xFFFFu;
            s1 = x >> 16;
            break;
        case 2:
            s0 = __builtin_amdgcn_ubfe(x, 12, 16);
            s1 = __builtin_amdgcn_ubfe(x, 8, 16);
            break;
        default:
            s0 = __builtin_amdgcn_ubfe(x, 4, 16);
            s1 = x & 0xFFFFu;
            break;
    }
    return PfPair{s0 * MCG_MUL, s1 * MCG_MUL};
}
__device__ __forceinline__ uint32_t pf_pair_values(PfPair m) {
    const uint32_t x0 = (m.x0 & MCG_MASK) ^ MCG_FLIP, x1 = (m.x1 & MCG_MASK) ^ MCG_FLIP;
    uint32_t d;
    asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1"
        : "=v"(d) : "v"(x0));
    asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1"
        : "+v"(d) : "v"(x1));
    return d;
}

__device__ __forceinline__ uint32_t pf_decode_pair(const uint32_t (&w)[3], int p) {
    const uint32_t pw = w[p >> 2], x = w[(p >> 2) + 1];
    uint32_t s0, s1;
    switch (p & 3) {
        case 0: {
            const uint32_t D = __builtin_amdgcn_alignbit(pw, x, 20);
            s0 = __builtin_amdgcn_ubfe(D, 8, 16);
            s1 = __builtin_amdgcn_ubfe(D, 4, 16);
            break;
        }
        case 1:
            s0 = __builtin_amdgcn_alignbit(pw, x, 20) & 0xFFFFu;
            s1 = x >> 16;
            break;
        case 2:
            s0 = __builtin_amdgcn_ubfe(x, 12, 16);
            s1 = __builtin_amdgcn_ubfe(x, 8, 16);
            break;
        default:
            s0 = __builtin_amdgcn_ubfe(x, 4, 16);
            s1 = x & 0xFFFFu;
            break;
    }
    // x = (s * MCG_MUL & MCG_MASK) ^ MCG_FLIP; value = fp16(x.lo) + fp16(x.hi), the pair's two values written to
    // the low and high halves of one register by two SDWA adds (the second preserves the first)
    const uint32_t x0 = ((s0 * MCG_MUL) & MCG_MASK) ^ MCG_FLIP, x1 = ((s1 * MCG_MUL) & MCG_MASK) ^ MCG_FLIP;
    uint32_t d;
    asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:WORD_0 src1_sel:WORD_1"
        : "=v"(d) : "v"(x0));
    asm("v_add_f16_sdwa %0, %1, %1 dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:WORD_0 src1_sel:WORD_1"
        : "+v"(d) : "v"(x1));
    return d;
}

// Staging, PF_NS steps of 16 PF_KT k deep, entirely by LDS DMA (global_load_lds_dwordx4): per step every wave copies
// 64 A rows (1 KB instructions, swizzled through the source addresses) and its own raw trellis words (PF_KT k tiles x
// 4 column tiles). Step it + PF_NS - 1 is issued while step it is multiplied, so each load has PF_NS - 1 steps of MFMA
// work to arrive; loads past the last step re-read it. The B operands of step it + 1 are decoded in registers during
// step it (no LDS round trip: each wave decodes only its own columns). One wait + barrier per step publishes A(it)
// (all waves) and the raw words of step it + 1 (this wave).
// E4M3: every decoded weight is rounded to the nearest e4m3 value (kept as the fp16 of that value), the trellis-
// sourced e4m3 variant's operand; the products with e4m3 activations are then exact and summed in fp32.
// NRB: the 32-row blocks of the tile that are multiplied (a compile-time count: tiles of up to 32 NRB rows skip the
// MFMAs and A reads of the other blocks, whose accumulators stay zero and are never stored; the decode is the same).
// TM: the A rows staged per step (256; 128 or 64 for the mid- and small-tile kernels). NS: staged steps (loads of
// step it + NS - 1 are issued while step it is multiplied).
template <bool E4M3 = false, int NRB = 8, int TM = PF_TM, int NS = PF_NS, bool ACOH = false>
__device__ __forceinline__ void pf_gemm(const PfTile& t, unsigned char* smem, f16v (&acc)[8][2]) {
    static_assert(32 * NRB <= TM && TM % 32 == 0, "the multiplied row blocks are staged");
    constexpr int ASB = TM * PF_RB;                                   // one A stage
    constexpr int CPR = PF_RB / 16;                                   // 16-byte chunks per A row
    constexpr int RPW = TM / 4;                                       // A rows staged by each wave
    constexpr int RPI = 64 / CPR;                                     // A rows per DMA instruction
    constexpr int NA = RPW / RPI;                                     // A DMA instructions per wave per step
    constexpr int NDMA = NA + PF_KT / 2;                              // DMA instructions per wave per step
    unsigned char* Ast = smem;                                        // [NS][TM rows][PF_RB]
    unsigned char* Wst = smem + NS * ASB;                          // [NS][4 waves][PF_KT k tiles][4 tiles][128 B]
    const int tid = opaque_tid(), lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int steps = t.kdim / (16 * PF_KT);
    // A DMA sources: instruction i of this wave = rows RPW wv + RPI i + lane / CPR, slot lane % CPR
    const uint16_t* asrc[NA];
#pragma unroll
    for (int i = 0; i < NA; ++i) {
        const int R = RPW * wv + RPI * i + lane / CPR;
        const int chunk = (lane % CPR) ^ pf_swz(R);
        const int rr = min(R, t.rn - 1);
        asrc[i] = t.a_rows + (size_t)(t.a_tok ? t.a_tok[rr] : rr) * t.kdim + 8 * chunk;
    }
    // raw-word DMA sources: instruction i, lane -> k tile 2i + lane / 32, column tile (lane / 8) % 4, piece lane % 8
    const uint32_t* wsrc = t.btr + ((size_t)(lane >> 5) * t.btiles_n + t.bcol0 + ((lane >> 3) & 3)) * 32 + 4 * (lane & 7);
    const size_t wstep = (size_t)PF_KT * t.btiles_n * 32;             // words per step (PF_KT k tiles)
    const size_t wins = (size_t)2 * t.btiles_n * 32;                  // words between a wave's W instructions
    auto issue_w = [&](int sw) {
        unsigned char* wd = Wst + (sw % NS) * PF_WSB + wv * PF_WWB;
#pragma unroll
        for (int i = 0; i < PF_KT / 2; ++i) dma16(wsrc + (size_t)sw * wstep + i * wins, wd + i * 1024);
    };
    auto issue_one = [&](int k, int sa, int sw) {                     // DMA instruction k of the batch (A(sa), W(sw))
        sa = min(sa, steps - 1);
        sw = min(sw, steps - 1);
        if (k < NA && ACOH)
            dma16_coh(asrc[k] + (size_t)sa * 16 * PF_KT, Ast + (sa % NS) * ASB + wv * RPW * PF_RB + k * 1024);
        else if (k < NA)
            dma16(asrc[k] + (size_t)sa * 16 * PF_KT, Ast + (sa % NS) * ASB + wv * RPW * PF_RB + k * 1024);
        else
            dma16(wsrc + (size_t)sw * wstep + (k - NA) * wins, Wst + (sw % NS) * PF_WSB + wv * PF_WWB + (k - NA) * 1024);
    };
    auto issue = [&](int sa, int sw) {                                // the whole batch
#pragma unroll
        for (int k = 0; k < NDMA; ++k) issue_one(k, sa, sw);
    };
    auto words = [&](int sw, uint32_t (&w)[PF_KT][3]) {              // this lane's raw words of step sw
        const unsigned char* wr = Wst + (sw % NS) * PF_WSB + wv * PF_WWB;
#pragma unroll
        for (int kt = 0; kt < PF_KT; ++kt) pf_load_words(wr + kt * 512, lane, w[kt]);
    };
    auto operands = [&](uint32_t (&q)[PF_KT][8], h8 (&b)[PF_KT][2]) {   // decoded pairs -> B operands
#pragma unroll
        for (int kt = 0; kt < PF_KT; ++kt) {
            if (E4M3) {
#pragma unroll
                for (int p = 0; p < 8; ++p) q[kt][p] = e4m3_round_h2(q[kt][p]);
            }
            b[kt][0] = __builtin_bit_cast(h8, u32x4{q[kt][0], q[kt][1], q[kt][4], q[kt][5]});
            b[kt][1] = __builtin_bit_cast(h8, u32x4{q[kt][2], q[kt][3], q[kt][6], q[kt][7]});
        }
    };
    auto afrag = [&](const unsigned char* as, int i) {                // A fragment i = (k tile i / 8, rows 32 (i % 8))
        const int R = 32 * (i & 7) + (lane & 31);
        const int slot = (2 * (i >> 3) + (lane >> 5)) ^ pf_swz(R);
        return *reinterpret_cast<const h8*>(as + R * PF_RB + 16 * slot);
    };
    // One step, in a fixed instruction order (one wave per SIMD issues everything itself): the 16 PF_KT MFMAs of
    // step it, each pair with one fp16 pair's decode for step it + 1 between them (VALU work issued while the MFMAs
    // run), the A fragments read four MFMA pairs ahead.
    constexpr int NF = 8 * PF_KT;                                     // A fragments (and decoded pairs) per step
    constexpr int DMA_EVERY = NF / NDMA;                              // MFMA pairs between DMA instructions
    auto step = [&](int it, const h8 (&bc)[PF_KT][2], h8 (&bn)[PF_KT][2]) {
        WAIT_VM(NDMA * (NS - 2));                                  // A(it) and words(it + 1): the oldest batch
        LDS_BARRIER();
        __builtin_amdgcn_sched_barrier(0);
        const unsigned char* as = Ast + (it % NS) * ASB;
        uint32_t w[PF_KT][3];
        words(it + 1, w);                                             // step it + 1 (past the end: never used)
        h8 af[NF];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            if (i < NRB) af[i] = afrag(as, i);
        __builtin_amdgcn_sched_barrier(0);
        uint32_t q[PF_KT][8];
        PfPair prev{0u, 0u};
#pragma unroll
        for (int i = 0; i < NF; ++i) {
            // the next batch's DMA instructions spread over the step (the CU's address path takes them one at a
            // time; issued together after the barrier they would stall every wave behind each other)
            if (i % DMA_EVERY == 0 && i / DMA_EVERY < NDMA) issue_one(i / DMA_EVERY, it + NS - 1, it + NS);
            if (i + 4 < NF && ((i + 4) & 7) < NRB) af[i + 4] = afrag(as, i + 4);
            const int kt = i >> 3, rb = i & 7;
            // pair i's products after the first MFMA, pair i - 1's values after the second: no VALU instruction
            // waits on the one before it while the MFMAs run
            if (rb < NRB) acc[rb][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bc[kt][0], acc[rb][0], 0, 0, 0);
            const PfPair cur = pf_pair_products(w[kt], i & 7);
            if (rb < NRB) acc[rb][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bc[kt][1], acc[rb][1], 0, 0, 0);
            if (i > 0) q[(i - 1) >> 3][(i - 1) & 7] = pf_pair_values(prev);
            prev = cur;
            __builtin_amdgcn_sched_barrier(0);
        }
        q[PF_KT - 1][7] = pf_pair_values(prev);
        operands(q, bn);
    };
#pragma unroll
    for (int rb = 0; rb < 8; ++rb)
#pragma unroll
        for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[rb][s][r] = 0.f;
    // prologue: raw words of step 0 first, then the batches that steps 0 .. NS - 2 of the loop would have issued
    // (A(0 .. NS - 2), words(1 .. NS - 1)); decode step 0
    issue_w(0);
#pragma unroll
    for (int j = 0; j < NS - 1; ++j) issue(j, j + 1);
    WAIT_VM(NDMA * (NS - 1));                                      // the step-0 words (this wave's own)
    h8 bA[PF_KT][2], bB[PF_KT][2];
    {
        uint32_t w[PF_KT][3], q[PF_KT][8];
        words(0, w);
#pragma unroll
        for (int i = 0; i < NF; ++i) q[i >> 3][i & 7] = pf_decode_pair(w[i >> 3], i & 7);
        operands(q, bA);
    }
    static_assert(NDMA * (NS - 1) <= 63 && PF_KT % 2 == 0, "stages within the vmcnt range");
    for (int it = 0; it < steps; it += 2) {                           // steps is even (kdim % (32 PF_KT) == 0)
        step(it, bA, bB);
        step(it + 1, bB, bA);
    }
    WAIT_VM(0);                                                       // nothing in flight when LDS is reused
    LDS_BARRIER();
}

// Stage the accumulators of row block rb (32 rows x 256 columns of the tile) into Cs [32][PF_CLD] fp32.
__device__ __forceinline__ void pf_stage_rows(const f16v (&acc)[8][2], float* Cs, int rb) {
    const int lane = opaque_tid() & 63;
    const int wv = __builtin_amdgcn_readfirstlane(opaque_tid() >> 6);
    const int n = lane & 31;
    const int col = 64 * wv + 16 * (n >> 3) + (n & 7);
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            Cs[row * PF_CLD + col + 8 * s] = acc[rb][s][r];
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

// The segments a launch takes: [lo, hi) = chunk `chunk` of `nchunks` equal shares of the live segments (all of them
// with one chunk; the reference's chunked schedule, code/fork/kernels/moe_e4m3.cu:479-481), never past the S_cap
// table entries. A grid's virtual segment s is segment lo + s.
__device__ __forceinline__ void pf_seg_range(const PrefillArgs& a, int& lo, int& hi) {
    const int ns = min(a.nseg[0], a.S_cap);
    if (a.nchunks <= 1) {
        lo = 0;
        hi = ns;
        return;
    }
    lo = (int)((int64_t)ns * a.chunk / a.nchunks);
    hi = (int)((int64_t)ns * (a.chunk + 1) / a.nchunks);
}

// ------------------------------------------------------------------------------------------------ gate/up

// E4M3: the trellis-sourced e4m3 variant (weights rounded to e4m3 in the GEMM; accumulators times the row's
// activation scale before the output Hadamard; the down input H(a16 * suh_d) * r kept in fp32 in vd, its row maxima
// gathered in amaxd for pf_quantd_kernel). code/fork/overlay/glm53_moe_e4m3.py:654-674 (spec_proj, spec_ffn).
// KIND: the tile is part `part` of the segment's rows in pf_sub_rows(KIND)-row parts (PF_LARGE: the whole segment).
template <bool E4M3, int KIND, bool COH = false>
__device__ __forceinline__ void pf_gateup_tile(const PrefillArgs& a, int s, int part, int cb, unsigned char* smem) {
    constexpr int SUB = pf_sub_rows(KIND);
    const int e = a.seg_expert[s];
    int row0 = a.seg_row0[s], rn = min(a.seg_rows[s], PF_TM);
    if (KIND != PF_LARGE) {
        row0 += SUB * part;
        rn = min(rn - SUB * part, SUB);
    }
    if (rn <= 0 || row0 < 0 || row0 + rn > a.P || e < 0 || e >= a.n) return;   // (caller-built tables)
    const int K = a.K, N = a.N;
    const int wv = __builtin_amdgcn_readfirstlane(opaque_tid() >> 6);
    PfTile t;                                                        // waves 0, 1: gate columns; 2, 3: up columns
    t.a_rows = a.tok_rows ? a.h13 : a.h13 + (size_t)row0 * K;       // tok_rows: the rows' tokens index h13
    t.a_tok = a.tok_rows ? a.tok + row0 : nullptr;
    t.rn = rn;
    t.kdim = K;
    t.btr = reinterpret_cast<const uint32_t*>(wv < 2 ? a.wt.g_tr[e] : a.wt.u_tr[e]);
    t.btiles_n = N >> 4;
    t.bcol0 = cb * 8 + 4 * (wv & 1);
    f16v acc[8][2];
    if (KIND == PF_SMALL) pf_gemm<E4M3, 2, PF_TMS>(t, smem, acc);
    else if (KIND == PF_MID && rn <= 64) pf_gemm<E4M3, 2, PF_TMM, PF_NSM>(t, smem, acc);
    else if (KIND == PF_MID) pf_gemm<E4M3, 4, PF_TMM, PF_NSM>(t, smem, acc);
    else if (rn <= 64) pf_gemm<E4M3, 2>(t, smem, acc);              // uniform: small tiles multiply two row blocks
    else pf_gemm<E4M3, 8>(t, smem, acc);

    // epilogue, 32 rows at a time through LDS; a wave finishes 4 rows at once: 16 lanes per row, lane c holding
    // columns 8c .. 8c + 7 (the 128-point Hadamards run across the 16 lanes by DPP)
    float* Cs = reinterpret_cast<float*>(smem);
    const int lane = opaque_tid() & 63;
    const int c = lane & 15, rsub = lane >> 4;
    const int col = cb * 128 + 8 * c;
    float svg[8], svu[8];
    _Float16 sud[8];
    // no down suh table: the SwiGLU output (a16out) is the epilogue's only output
    const _Float16* dsp = a.wt.d_suh ? reinterpret_cast<const _Float16*>(a.wt.d_suh[e]) : nullptr;
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
        const h2 g2 = *reinterpret_cast<const h2*>(reinterpret_cast<const _Float16*>(a.wt.g_svh[e]) + col + i);
        const h2 u2 = *reinterpret_cast<const h2*>(reinterpret_cast<const _Float16*>(a.wt.u_svh[e]) + col + i);
        const h2 d2 = dsp ? *reinterpret_cast<const h2*>(dsp + col + i) : h2{(_Float16)1.0f, (_Float16)1.0f};
        svg[i] = (float)g2.x, svg[i + 1] = (float)g2.y;
        svu[i] = (float)u2.x, svu[i + 1] = (float)u2.y;
        sud[i] = d2.x, sud[i + 1] = d2.y;
    }
    // storage of the lane's pairs m = 0..3 (columns 8c + 2m, + 1): k pair j = 4 (c % 2) + m of group c / 2
    const int grp0 = cb * 128 + 16 * (c >> 1);                      // the lane's 16-group of the block
    const float L = a.limit;
    const float hr = HAD_R * fwht_sign(lane);                        // r and the sign fwht128_x16s leaves
    // E4M3: the activation scales of the rows this lane's passes take (block rb, pass p: row 32 rb + 8 wv + 4 p +
    // rsub), loaded in one batch (token ids, then scales) instead of two dependent loads per pass
    float rsc[SUB / 32][2];
    if (E4M3) {
        int ri[SUB / 32][2];
#pragma unroll
        for (int rb = 0; rb < SUB / 32; ++rb)
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const int ar = row0 + min(32 * rb + wv * 8 + p * 4 + rsub, rn - 1);
                ri[rb][p] = a.tok_rows ? a.tok[ar] : ar;
            }
#pragma unroll
        for (int rb = 0; rb < SUB / 32; ++rb)
#pragma unroll
            for (int p = 0; p < 2; ++p) rsc[rb][p] = a.asc[ri[rb][p]];
    }
    // RBS row blocks are staged per pair of barriers (as many as the kernel's LDS holds), so each wave runs 2 RBS
    // row passes of independent work between barriers
    constexpr int RBS = pf_epi_blocks(KIND);
#pragma unroll
    for (int rb0 = 0; rb0 < SUB / 32; rb0 += RBS) {
        if (32 * rb0 >= rn) break;                                   // uniform over the workgroup
#pragma unroll
        for (int q = 0; q < RBS; ++q)
            if (rb0 + q < SUB / 32 && 32 * (rb0 + q) < rn) pf_stage_rows(acc, Cs + q * 32 * PF_CLD, rb0 + q);
        __syncthreads();
#pragma unroll
        for (int q = 0; q < RBS; ++q) {
            const int rb = rb0 + q;
            if (rb >= SUB / 32 || 32 * rb >= rn) continue;             // uniform
            // the block's two row passes at once (rows 4 p + rsub of each wave's 8, p = 0, 1): two rows per 16-lane
            // group, so every Hadamard stage has four (then two) independent vectors of work
            int trow[2];
            float gu[4][8], b[2][8];                                  // gu: g of rows 0, 1, then u of rows 0, 1
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const int rl = wv * 8 + p * 4 + rsub;
                trow[p] = 32 * rb + rl;
                const float* cr = Cs + (q * 32 + rl) * PF_CLD + 8 * c;
#pragma unroll
                for (int i = 0; i < 8; i += 4) {
                    const float4 g4 = *reinterpret_cast<const float4*>(cr + i);
                    const float4 u4 = *reinterpret_cast<const float4*>(cr + 128 + i);
                    gu[p][i] = g4.x, gu[p][i + 1] = g4.y, gu[p][i + 2] = g4.z, gu[p][i + 3] = g4.w;
                    gu[2 + p][i] = u4.x, gu[2 + p][i + 1] = u4.y, gu[2 + p][i + 2] = u4.z, gu[2 + p][i + 3] = u4.w;
                }
                if (E4M3) {                                          // dequantise: times the row's activation scale
                    const float rs = rsc[rb][p];
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        gu[p][i] *= rs;
                        gu[2 + p][i] *= rs;
                    }
                }
            }
            fwht128_x16s_n<4>(gu, lane);
            _Float16 av[2][8];
#pragma unroll
            for (int p = 0; p < 2; ++p)
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    float gv = gu[p][i] * hr * svg[i];
                    float uv = gu[2 + p][i] * hr * svu[i];
                    if (L != 0.0f) {
                        gv = fminf(gv, L);
                        uv = fminf(fmaxf(uv, -L), L);
                    }
                    av[p][i] = (_Float16)(sigmoid_fast(gv) * gv * uv);
                    b[p][i] = E4M3 ? (float)av[p][i] * (float)sud[i] : (float)(_Float16)(av[p][i] * sud[i]);
                }
            if (E4M3 && a.a16out) {                                  // the fp16 SwiGLU output, plain column order
#pragma unroll
                for (int p = 0; p < 2; ++p)
                    if (trow[p] < rn)
                        *reinterpret_cast<h8*>(a.a16out + (size_t)(row0 + trow[p]) * N + col) =
                            h8{av[p][0], av[p][1], av[p][2], av[p][3], av[p][4], av[p][5], av[p][6], av[p][7]};
            }
            if (E4M3 && !a.down16 && !a.vd) continue;                // (uniform) a16 was the only output
            fwht128_x16s_n<2>(b, lane);
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                if (E4M3 && !a.down16) {                             // fp32 down input and its row maximum
                    float m = 0.0f;
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        b[p][i] = b[p][i] * hr;
                        m = fmaxf(m, fabsf(b[p][i]));
                    }
                    m = fmaxf(m, xor_lane<1>(m, lane));
                    m = fmaxf(m, xor_lane<2>(m, lane));
                    m = fmaxf(m, xor_lane<4>(m, lane));
                    m = fmaxf(m, xor_lane<8>(m, lane));
                    if (trow[p] < rn) {
                        float* vo = a.vd + (size_t)(row0 + trow[p]) * N + col;
                        if (COH) {                           // buffer over the tile's rows (row0: uniform)
                            const __amdgpu_buffer_rsrc_t rv = coh_rsrc(a.vd + (size_t)row0 * N);
                            const int off = 4 * (trow[p] * N + col);
                            st_coh16(rv, off, __builtin_bit_cast(u32x4, f32x4{b[p][0], b[p][1], b[p][2], b[p][3]}));
                            st_coh16(rv, off + 16, __builtin_bit_cast(u32x4, f32x4{b[p][4], b[p][5], b[p][6], b[p][7]}));
                        } else {
                            *reinterpret_cast<float4*>(vo) = make_float4(b[p][0], b[p][1], b[p][2], b[p][3]);
                            *reinterpret_cast<float4*>(vo + 4) = make_float4(b[p][4], b[p][5], b[p][6], b[p][7]);
                        }
                        if (c == 0) atomicMax(a.amaxd + row0 + trow[p], __builtin_bit_cast(unsigned, m));
                    }
                } else {
                    uint32_t wm[4];
#pragma unroll
                    for (int m = 0; m < 4; ++m)
                        wm[m] = __builtin_bit_cast(uint32_t,
                                                   h2{(_Float16)(b[p][2 * m] * hr), (_Float16)(b[p][2 * m + 1] * hr)});
                    if (trow[p] < rn) {
                        if (COH)
                            pf_store_group_coh(coh_rsrc(reinterpret_cast<_Float16*>(a.h2) + (size_t)row0 * N),
                                               2 * (trow[p] * N + grp0), wm, c);
                        else
                            pf_store_group(reinterpret_cast<_Float16*>(a.h2) + (size_t)(row0 + trow[p]) * N + grp0, wm, c);
                    }
                }
            }
        }
        __syncthreads();
    }
}

// Workgroup b of a grid of segment parts (8 ncb ceil(parts S_cap / 8) workgroups): tile (virtual segment v, column
// block cb) as pf_tile_of orders them, v = part S_cap + s, so the first parts of all segments come first and the
// later parts' workgroups, empty for segments of fewer rows, come last.
__device__ __forceinline__ bool pf_part_tile_of(const PrefillArgs& a, int ncb, int parts, int& s, int& part, int& cb) {
    int v, lo, hi;
    pf_tile_of(blockIdx.x, ncb, v, cb);
    if (a.S_cap <= 0 || v >= parts * a.S_cap) return false;
    part = v / a.S_cap;
    s = v - part * a.S_cap;
    pf_seg_range(a, lo, hi);
    s += lo;
    return s < hi;
}

template <bool E4M3>
__global__ __launch_bounds__(PF_THREADS, 1) void pf_gateup_kernel(PrefillArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    int s, cb, lo, hi;
    pf_tile_of(blockIdx.x, a.N >> 7, s, cb);
    pf_seg_range(a, lo, hi);
    s += lo;
    if (s >= hi || (a.small_rows > 0 && a.seg_rows[s] <= a.small_rows)) return;
    pf_gateup_tile<E4M3, PF_LARGE>(a, s, 0, cb, smem);
}

// The same GEMM for segments of few rows: 64-row tiles with 64 KB of LDS and at most 256 registers per wave, so two
// workgroups share a CU and one's waits are covered by the other's work (a tile's weight decode does not shrink
// with its rows, so at ~60 rows per expert the decode, not the MFMA, bounds the GEMM).
template <bool E4M3>
__global__ __launch_bounds__(PF_THREADS) __attribute__((amdgpu_waves_per_eu(2))) void pf_gateup_small_kernel(
    PrefillArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    int s, quarter, cb;
    if (!pf_part_tile_of(a, a.N >> 7, 4, s, quarter, cb)) return;
    if (a.small_rows > 0 && a.seg_rows[s] > a.small_rows) return;
    pf_gateup_tile<E4M3, PF_SMALL>(a, s, quarter, cb, smem);
}

// The same GEMM on 128-row halves of the segments (73,728 bytes of LDS in three stages, at most 256 registers per
// wave, two workgroups per CU): each weight is decoded twice per 256-row segment, and one workgroup's epilogue and
// waits are covered by the other's main loop.
template <bool E4M3>
__global__ __launch_bounds__(PF_THREADS) __attribute__((amdgpu_waves_per_eu(2))) void pf_gateup_mid_kernel(
    PrefillArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    int s, half, cb;
    if (!pf_part_tile_of(a, a.N >> 7, 2, s, half, cb)) return;
    pf_gateup_tile<E4M3, PF_MID>(a, s, half, cb, smem);
}

// ------------------------------------------------------------------------------------------------ down

template <bool E4M3, int KIND, bool ACOH = false>
__device__ __forceinline__ void pf_down_tile(const PrefillArgs& a, int s, int part, int cb, unsigned char* smem) {
    constexpr int SUB = pf_sub_rows(KIND);
    const int e = a.seg_expert[s];
    int row0 = a.seg_row0[s], rn = min(a.seg_rows[s], PF_TM);
    if (KIND != PF_LARGE) {
        row0 += SUB * part;
        rn = min(rn - SUB * part, SUB);
    }
    if (rn <= 0 || row0 < 0 || row0 + rn > a.P || e < 0 || e >= a.n) return;   // (caller-built tables)
    const int K = a.K, N = a.N;
    const int wv = __builtin_amdgcn_readfirstlane(opaque_tid() >> 6);
    PfTile t;
    t.a_rows = a.h2 + (size_t)row0 * N;
    t.a_tok = nullptr;
    t.rn = rn;
    t.kdim = N;
    t.btr = reinterpret_cast<const uint32_t*>(a.wt.d_tr[e]);
    t.btiles_n = K >> 4;
    t.bcol0 = cb * 16 + 4 * wv;
    f16v acc[8][2];
    if (KIND == PF_SMALL) pf_gemm<E4M3, 2, PF_TMS>(t, smem, acc);
    else if (KIND == PF_MID && rn <= 64) pf_gemm<E4M3, 2, PF_TMM, PF_NSM>(t, smem, acc);
    else if (KIND == PF_MID) pf_gemm<E4M3, 4, PF_TMM, PF_NSM>(t, smem, acc);
    else if (rn <= 64) pf_gemm<E4M3, 2, PF_TM, PF_NS, ACOH>(t, smem, acc);
    else pf_gemm<E4M3, 8, PF_TM, PF_NS, ACOH>(t, smem, acc);

    // epilogue: the raw accumulators (rows < rn) straight from registers into contrib; the output rotation, svh and
    // router weight are applied by the combine (the VALU work runs there, beside its memory traffic, instead of after
    // this kernel's MFMAs). Lane n of block s holds column 16 (n / 8) + n % 8 + 8 s of the wave.
    const int lane = opaque_tid() & 63;
    const int n = lane & 31;
    const size_t c0 = (size_t)row0 * K + cb * 256 + 64 * wv + 16 * (n >> 3) + (n & 7);
    // row blocks wholly inside the segment store unguarded (uniform test); only the block holding row rn is masked
    if (a.contrib_bf16) {
        // bf16 raw accumulators: lane n holds columns c (block 0) and c + 8 (block 1), its partner n ^ 1 columns
        // c + 1 and c + 9 (n even). Each lane packs its own two values, takes the partner's pack (DPP lane ^ 1) and
        // keeps one column pair: the even lane (c, c + 1), the odd lane (c + 8, c + 9), one 4-byte store each.
        uint16_t* ob = reinterpret_cast<uint16_t*>(a.contrib) + c0 + ((n & 1) ? 7 : 0);
        const uint32_t sel = (n & 1) ? 0x03020706u : 0x05040100u;  // bytes of {partner, own}: odd hi halves, even lo
        auto put = [&](int rb, int r) {
            const int trow = 32 * rb + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            const uint32_t own = pack_bf16x2(acc[rb][0][r], acc[rb][1][r]);
            const uint32_t par = (uint32_t)__builtin_amdgcn_mov_dpp((int)own, 0xB1, 0xF, 0xF, true);
            return std::pair<uint32_t*, uint32_t>(reinterpret_cast<uint32_t*>(ob + (size_t)trow * K),
                                                  __builtin_amdgcn_perm(par, own, sel));
        };
#pragma unroll
        for (int rb = 0; rb < SUB / 32; ++rb) {
            if (32 * rb >= rn) break;
            if (32 * rb + 32 <= rn) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const auto pv = put(rb, r);
                    *pv.first = pv.second;
                }
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const auto pv = put(rb, r);                       // (the DPP runs with every lane active)
                    if (32 * rb + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3) < rn) *pv.first = pv.second;
                }
            }
        }
        return;
    }
    // fp32: lane n holds columns c and c + 8, its partner n ^ 1 columns c + 1 and c + 9 (n even). The pair trades one
    // value (DPP lane ^ 1) so that the even lane stores (c, c + 1) and the odd lane (c + 8, c + 9), 8 bytes each.
    const bool odd = n & 1;
    float* o = a.contrib + c0 + (odd ? 7 : 0);
    auto pair = [&](int rb, int r) {
        const float v0 = acc[rb][0][r], v1 = acc[rb][1][r];          // (values first: a select of addresses
        const float send = odd ? v0 : v1;                             //  would send the array to scratch)
        const float recv = __builtin_bit_cast(
            float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, send), 0xB1, 0xF, 0xF, true));
        return make_float2(odd ? recv : v0, odd ? v1 : recv);
    };
#pragma unroll
    for (int rb = 0; rb < SUB / 32; ++rb) {
        if (32 * rb >= rn) break;
        if (32 * rb + 32 <= rn) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int trow = 32 * rb + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                *reinterpret_cast<float2*>(o + (size_t)trow * K) = pair(rb, r);
            }
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int trow = 32 * rb + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const float2 v = pair(rb, r);                          // (the DPP runs with every lane active)
                if (trow < rn) *reinterpret_cast<float2*>(o + (size_t)trow * K) = v;
            }
        }
    }
}

template <bool E4M3>
__global__ __launch_bounds__(PF_THREADS, 1) void pf_down_kernel(PrefillArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    int s, cb, lo, hi;
    pf_tile_of(blockIdx.x, a.K >> 8, s, cb);
    pf_seg_range(a, lo, hi);
    s += lo;
    if (s >= hi || (a.small_rows > 0 && a.seg_rows[s] <= a.small_rows)) return;
    pf_down_tile<E4M3, PF_LARGE>(a, s, 0, cb, smem);
}

template <bool E4M3>
__global__ __launch_bounds__(PF_THREADS) __attribute__((amdgpu_waves_per_eu(2))) void pf_down_small_kernel(
    PrefillArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    int s, quarter, cb;
    if (!pf_part_tile_of(a, a.K >> 8, 4, s, quarter, cb)) return;
    if (a.small_rows > 0 && a.seg_rows[s] > a.small_rows) return;
    pf_down_tile<E4M3, PF_SMALL>(a, s, quarter, cb, smem);
}

template <bool E4M3>
__global__ __launch_bounds__(PF_THREADS) __attribute__((amdgpu_waves_per_eu(2))) void pf_down_mid_kernel(
    PrefillArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    int s, half, cb;
    if (!pf_part_tile_of(a, a.K >> 8, 2, s, half, cb)) return;
    pf_down_tile<E4M3, PF_MID>(a, s, half, cb, smem);
}

// ------------------------------------------------------------------------------------------------ one-launch schedule

// Every gate/up and down tile of a call in one launch of one workgroup per CU (256-row tiles; two per CU for the
// 128- and 64-row part tiles, KIND below). The segments are dealt to eight ticket queues (segment s to queue s % 8, as the separate launches deal them to the
// XCDs), each ordered by pf_sched_item over its own segments; a workgroup takes tickets from its own XCD's queue
// (the XCC_ID register), so a segment's column blocks share that XCD's L2 for their A rows, and once that queue is
// empty from the other queues in turn. A gate/up item stores its h2 rows device-coherent (written through to the
// device coherence point, so no L2 write-back fence is needed), and once every wave's stores have completed
// (s_waitcnt, then a barrier) one lane raises the segment's count. A down item waits until the count reaches the
// segment's ncg gate/up items (one lane polls with agent-scope atomic loads, sleeping between polls) and loads the
// h2 rows device-coherent (so no cache invalidation is needed). The gate/up items a down item waits for have smaller
// tickets of the same queue, so running workgroups hold them, and they never wait themselves: every wait ends. A
// wait is still bounded (PF_SCHED_POLLS polls): one that runs out sets the give-up word, skips its tile, and every
// later wait gives up at once, so a broken table costs a wrong result, never a hung launch. The tiles run the
// separate launches' code on the same rows, so the results are bit-identical to theirs.
// MODE: PF_SCHED_E3 (E3 numerics), PF_SCHED_E4M3_16 (trellis-sourced e4m3 gate/up writing the fp16 down input h2,
// fp16 down GEMM) or PF_SCHED_E4M3 (the e4m3 gate/up writes the fp32 down input vd and its row maxima amaxd, both
// device-coherent; the workgroup whose gate/up item completes a segment -- its count reaches ncg -- quantises the
// segment's rows to h2 and dsc (device-coherent) and adds one more, and the segment's down items, e4m3 GEMMs, wait
// for ncg + 1: the reference's dataflow, code/fork/kernels/moe_e4m3.cu:867-872).
enum { PF_SCHED_E3 = 0, PF_SCHED_E4M3_16 = 1, PF_SCHED_E4M3 = 2 };
constexpr int PF_SCHED_POLLS = 1 << 20;
// KIND: the call's tile kind (PF_LARGE: 256-row segments, one workgroup per CU; PF_MID / PF_SMALL: the segments'
// 128- or 64-row parts, two workgroups per CU). A queue's units are its (segment, part) pairs, every segment's first
// part first; a part past its segment's rows holds no tile, so its items only take their tickets. Each unit has its
// own count (segment s, part p: word PF_SCHED_HEAD + s * parts + p).
template <int MODE, int KIND>
__device__ __forceinline__ void pf_sched_body(const PrefillArgs& a, unsigned char* smem) {
    constexpr int PARTS = KIND == PF_SMALL ? 4 : KIND == PF_MID ? 2 : 1;
    constexpr int SUB = pf_sub_rows(KIND);
    // The item's ticket and whether its wait ran out sit in the first LDS words between tiles (the tiles' stages
    // take the whole LDS): written by one lane, read by every wave after a barrier, and overwritten by the tile's
    // loads only after a second barrier.
    int* s_ctl = reinterpret_cast<int*>(smem);
    int lo, hi;
    pf_seg_range(a, lo, hi);
    const int ns = hi - lo, ncg = a.N >> 7, ncd = a.K >> 8;
    const int ready_at = ncg + (MODE == PF_SCHED_E4M3 ? 1 : 0);      // a down item's unit count to wait for
    int* ctl = a.sched;
    int* gave_up_word = ctl + PF_SCHED_QUEUES * PF_SCHED_QSTRIDE;
    int* ready = ctl + PF_SCHED_HEAD;
    const int xq = __builtin_amdgcn_s_getreg((2 << 11) | 20) & (PF_SCHED_QUEUES - 1);   // XCC_ID bits 2:0
    for (int d = 0; d < PF_SCHED_QUEUES; ++d) {
        const int q = (xq + d) & (PF_SCHED_QUEUES - 1);
        const int nq = ns > q ? (ns - q + PF_SCHED_QUEUES - 1) / PF_SCHED_QUEUES : 0;   // the queue's segments
        int* ticket = ctl + q * PF_SCHED_QSTRIDE;
        while (nq > 0) {
            WAIT_VM(0);                                               // the last item's stores have completed
            __syncthreads();                                          // and every wave is done with LDS
            if (threadIdx.x == 0) {
                s_ctl[0] = __hip_atomic_fetch_add(ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                s_ctl[1] = 0;
            }
            __syncthreads();
            const PfSchedItem it =
                pf_sched_item(__builtin_amdgcn_readfirstlane(s_ctl[0]), nq * PARTS, a.sched_lag, ncg, ncd);
            if (it.kind < 0) break;                                   // (uniform) the queue is empty
            const int part = it.seg / nq, s = lo + q + PF_SCHED_QUEUES * (it.seg - part * nq);   // s < hi
            if (PARTS > 1 && __builtin_amdgcn_readfirstlane(a.seg_rows[s]) <= SUB * part) continue;   // no tile
            int* cnt = ready + s * PARTS + part;
            if (it.kind == 0) {
                __syncthreads();                                      // every wave has read s_ctl
                // h2 (or vd and amaxd) stored device-coherent
                pf_gateup_tile<MODE != PF_SCHED_E3, KIND, true>(a, s, part, it.block, smem);
                WAIT_VM(0);                                           // this wave's stores have completed
                __syncthreads();
                if (MODE != PF_SCHED_E4M3) {
                    if (threadIdx.x == 0) __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    continue;
                }
                if (threadIdx.x == 0)
                    s_ctl[1] = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ncg - 1;
                __syncthreads();
                if (!__builtin_amdgcn_readfirstlane(s_ctl[1])) continue;   // (uniform) not the unit's last
                // the unit's last gate/up item: every other one's stores completed before its count; quantise the
                // unit's rows (one wave per row) and publish them with one more count
                const int r0 = a.seg_row0[s] + SUB * part, rn = min(a.seg_rows[s] - SUB * part, SUB);
                constexpr int QR = 4;                                 // rows in flight per wave
                const int w0 = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
                if (r0 >= 0 && rn > 0 && r0 + rn <= a.P) {           // (caller-built tables)
                    if (a.N <= 1024)
                        for (int r = w0; r < rn; r += QR * (PF_THREADS / 64))
                            pf_quantd_rows_coh<QR>(a, r0 + r, PF_THREADS / 64, r0 + rn, threadIdx.x & 63);
                    else
                        for (int r = w0; r < rn; r += PF_THREADS / 64) pf_quantd_row<true>(a, r0 + r, threadIdx.x & 63);
                }
                WAIT_VM(0);
                __syncthreads();
                if (threadIdx.x == 0) __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                continue;
            }
            if (threadIdx.x == 0) {
                for (int polls = 0; __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < ready_at;
                     ++polls) {
                    if (polls >= PF_SCHED_POLLS ||
                        __hip_atomic_load(gave_up_word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
                        __hip_atomic_store(gave_up_word, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        s_ctl[1] = 1;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(4);
                }
            }
            __syncthreads();
            const int gave_up = __builtin_amdgcn_readfirstlane(s_ctl[1]);
            __syncthreads();                                          // every wave has read s_ctl
            if (gave_up) continue;                                    // (uniform) the tile is skipped
            pf_down_tile<MODE == PF_SCHED_E4M3, KIND, true>(a, s, part, it.block, smem);   // h2 device-coherent
        }
    }
}
template <int MODE>
__global__ __launch_bounds__(PF_THREADS, 1) void pf_sched_kernel(PrefillArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    pf_sched_body<MODE, PF_LARGE>(a, smem);
}
template <int MODE, int KIND>
__global__ __launch_bounds__(PF_THREADS) __attribute__((amdgpu_waves_per_eu(2))) void pf_sched_part_kernel(
    PrefillArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    pf_sched_body<MODE, KIND>(a, smem);
}

// ------------------------------------------------------------------------------------------------ combine

// One wave per (token t, 512 columns): out[t] = sum over the token's slots k (in order) of the valid pairs'
// contributions ((H(acc) * r) * svh_d) * w16, in the output dtype (deterministic: no atomics). A 16-lane group
// rotates one 128-column block (lane c holding columns 8c .. 8c + 7, DPP Hadamard); the loads of eight slots (their
// raw rows and their experts' svh) are issued before the first rotation.
__global__ __launch_bounds__(256) void pf_combine_kernel(PrefillArgs a) {
    const int t = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * 4 + (threadIdx.x >> 6)));
    if (t >= a.T) return;
    const int lane = threadIdx.x & 63;
    const float hr = HAD_R * fwht_sign(lane);                        // r and the sign fwht128_x16s leaves
    const int col = blockIdx.y * 512 + 128 * (lane >> 4) + 8 * (lane & 15);
    const bool live = blockIdx.y * 512 + 128 * (lane >> 4) < a.K;    // whole 16-lane groups
    const int colc = live ? col : 0;
    float sum[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < a.topk; k0 += 8) {
        // lanes 0..7 fetch slot k0 + lane's position, expert and weight (one vector load each), broadcast by readlane
        const int lk = k0 + (lane & 7);
        const int pl = a.inv[t * a.topk + min(lk, a.topk - 1)];
        const int el = a.pe[pl];
        // thin/fat split: a row this path skipped but the decode kernels computed holds a finished contribution
        const int thl = (int)(lk < a.topk && el < 0 && a.pe_thin && a.pe_thin[pl] >= 0);
        const int okl = (int)(lk < a.topk) & (int)(el >= 0 || thl);
        const float wl = a.w32 ? a.w32[pl] : (float)u16_as_h(a.w16[pl]);
        const float dl = a.dsc ? a.dsc[pl] : 1.0f;                   // e4m3 variant: the down input's row scale
        const int64_t svl = a.wt.d_svh[max(el, 0)];
        f32x4 raw[8][2];
        u32x4 sv[8];
        bool ok[8], thin[8];
        float w[8], ds[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {                                 // unconditional loads (no joins between them)
            const int pos = __builtin_amdgcn_readlane(pl, k);
            ok[k] = __builtin_amdgcn_readlane(okl, k) != 0;
            thin[k] = __builtin_amdgcn_readlane(thl, k) != 0;
            w[k] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), k));
            ds[k] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, dl), k));
            const uint64_t sp = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)svl, k)) |
                                ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(svl >> 32), k) << 32);
            if (a.contrib_bf16) {                                    // 8 bf16 in the first vector's place
                const u32x4 rb16 = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(a.contrib) +
                                                                   (size_t)pos * a.K + colc);
                raw[k][0] = __builtin_bit_cast(f32x4, rb16);
            } else {
                const float* rp = a.contrib + (size_t)pos * a.K + colc;
                raw[k][0] = *reinterpret_cast<const f32x4*>(rp);
                raw[k][1] = *reinterpret_cast<const f32x4*>(rp + 4);
            }
            const uint16_t* svp = reinterpret_cast<const uint16_t*>(sp) + colc;
#pragma unroll
            for (int i = 0; i < 4; ++i) sv[k][i] = *reinterpret_cast<const uint32_t*>(svp + 2 * i);
        }
        bool any_thin = false;
#pragma unroll
        for (int k = 0; k < 8; ++k) any_thin |= thin[k];
        if (!any_thin) {                                             // (uniform) four slots' rotations at a time
#pragma unroll
            for (int k0h = 0; k0h < 8; k0h += 4) {
                float v[4][8];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int k = k0h + j;
                    if (a.contrib_bf16) {
                        const u32x4 rb16 = __builtin_bit_cast(u32x4, raw[k][0]);
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            v[j][2 * i] = bf16_to_f32((uint16_t)(rb16[i] & 0xFFFFu));
                            v[j][2 * i + 1] = bf16_to_f32((uint16_t)(rb16[i] >> 16));
                        }
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            v[j][i] = raw[k][0][i];
                            v[j][4 + i] = raw[k][1][i];
                        }
                    }
                    if (a.dsc) {
#pragma unroll
                        for (int i = 0; i < 8; ++i) v[j][i] *= ds[k];
                    }
                }
                fwht128_x16s_n<4>(v, lane);
#pragma unroll
                for (int j = 0; j < 4; ++j) {                        // slot order, as below
                    const int k = k0h + j;
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const uint32_t s2 = sv[k][i >> 1];
                        const float svf = (float)u16_as_h((i & 1) ? s2 >> 16 : s2 & 0xFFFFu);
                        if (ok[k]) sum[i] += v[j][i] * hr * svf * w[k];
                    }
                }
            }
            continue;
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            float v[8];
            if (a.contrib_bf16 && !thin[k]) {
                const u32x4 rb16 = __builtin_bit_cast(u32x4, raw[k][0]);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    v[2 * i] = bf16_to_f32((uint16_t)(rb16[i] & 0xFFFFu));
                    v[2 * i + 1] = bf16_to_f32((uint16_t)(rb16[i] >> 16));
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    v[i] = raw[k][0][i];
                    v[4 + i] = raw[k][1][i];
                }
            }
            if (thin[k]) {                                           // uniform: one slot per wave
#pragma unroll
                for (int i = 0; i < 8; ++i) sum[i] += v[i];
                continue;
            }
            if (a.dsc) {
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] *= ds[k];
            }
            fwht128_x16s(v, lane);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t s2 = sv[k][i >> 1];
                const float svf = (float)u16_as_h((i & 1) ? s2 >> 16 : s2 & 0xFFFFu);
                if (ok[k]) sum[i] += v[i] * hr * svf * w[k];
            }
        }
    }
    if (!live) return;
    const size_t o = (size_t)t * a.out_stride + col;
    if (a.out_accumulate) {                                          // out += the routed sum (one rounding)
        float prev[8];
        if (a.odt == DT_F32) {
#pragma unroll
            for (int i = 0; i < 8; ++i) prev[i] = reinterpret_cast<const float*>(a.out)[o + i];
        } else if (a.odt == DT_BF16) {
#pragma unroll
            for (int i = 0; i < 8; ++i) prev[i] = bf16_to_f32(reinterpret_cast<const uint16_t*>(a.out)[o + i]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) prev[i] = (float)reinterpret_cast<const _Float16*>(a.out)[o + i];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) sum[i] = prev[i] + sum[i];
    }
    if (a.odt == DT_F32) {
        float* op = reinterpret_cast<float*>(a.out) + o;
#pragma unroll
        for (int i = 0; i < 8; i += 2) *reinterpret_cast<float2*>(op + i) = make_float2(sum[i], sum[i + 1]);
    } else if (a.odt == DT_BF16) {
        uint32_t* op = reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(a.out) + o);
#pragma unroll
        for (int i = 0; i < 4; ++i) op[i] = pack_bf16x2(sum[2 * i], sum[2 * i + 1]);
    } else {
        h2* op = reinterpret_cast<h2*>(reinterpret_cast<uint16_t*>(a.out) + o);
#pragma unroll
        for (int i = 0; i < 4; ++i) op[i] = h2{(_Float16)sum[2 * i], (_Float16)sum[2 * i + 1]};
    }
}

// ------------------------------------------------------------------------------------------------ row-table down

// Rows of caller-built tables: pe[r] = -1 for every row and cnt[t] = 0 for every token, then pe[r] = the expert of the
// segment covering row r (segments s < nseg[0]); rows no segment covers stay skipped.
// tok32 (optional): tok32[r] = row_token[r] as int32, 0 where it lies outside [0, tokens).
__global__ __launch_bounds__(256) void pf_rows_init_kernel(PrefillArgs a, int* pe, int* cnt, int tokens, int* tok32,
                                                           const int64_t* row_token) {
    if (a.sched && blockIdx.x == 0)                                   // the one-launch schedule's control words
        for (int i = threadIdx.x; i < PF_SCHED_WORDS(a.S_cap); i += 256) a.sched[i] = 0;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < max(a.P, tokens); i += gridDim.x * 256) {
        if (i < a.P) {
            pe[i] = -1;
            if (a.amaxd) a.amaxd[i] = 0u;
            if (tok32) {
                const int64_t t = row_token[i];
                tok32[i] = (t >= 0 && t < tokens) ? (int)t : 0;
            }
        }
        if (i < tokens) cnt[i] = 0;
    }
}

// out[t][0 .. K) = 0 for t < T (fp32 or bf16, row stride out_stride): the zero fill of an accumulated output.
__global__ __launch_bounds__(256) void pf_zero_out_kernel(PrefillArgs a) {
    const int per = a.K / 8;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < (int64_t)a.T * per; i += (int64_t)gridDim.x * 256) {
        const int64_t t = i / per, c = 8 * (i % per);
        if (a.odt == DT_F32) {
            float* o = reinterpret_cast<float*>(a.out) + t * a.out_stride + c;
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = 0.0f;
        } else {
            uint16_t* o = reinterpret_cast<uint16_t*>(a.out) + t * a.out_stride + c;
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = 0;
        }
    }
}
// One workgroup per segment of the launch's range (pf_seg_range); with a.row_expert the rows are marked with their own
// row_expert entries (the segment's expert is not read).
__global__ __launch_bounds__(256) void pf_seg_rows_kernel(PrefillArgs a, int* pe) {
    int lo, hi;
    pf_seg_range(a, lo, hi);
    const int s = lo + (int)blockIdx.x;
    if (s >= hi) return;
    const int e = a.row_expert ? 0 : a.seg_expert[s], row0 = a.seg_row0[s], rn = min(a.seg_rows[s], PREFILL_TM);
    if (e < 0 || e >= a.n) return;                                    // (the GEMM kernels skip such segments too)
    for (int i = threadIdx.x; i < rn; i += 256)
        if (row0 + i >= 0 && row0 + i < a.P) pe[row0 + i] = a.row_expert ? a.row_expert[row0 + i] : e;
}

// e4m3 code rows (one byte per element, in the staging order of h13 / h2) widened to the fp16 staging rows the GEMMs
// read: dst[r][k] = the fp16 of the e4m3 value src[r][k] (exact: every e4m3 value is an fp16), for every row r < rows
// (pe == nullptr) or those with pe[r] >= 0. One wave per row, 16 codes per lane per pass; cols % 16 == 0.
__global__ __launch_bounds__(256) void pf_widen8_kernel(const uint8_t* __restrict__ src, uint16_t* __restrict__ dst,
                                                        int cols, int rows, const int* __restrict__ pe) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * 4 + (threadIdx.x >> 6)));
    for (int r = wave; r < rows; r += gridDim.x * 4) {
        if (pe && pe[r] < 0) continue;                               // uniform: one row per wave
        const uint8_t* sr = src + (size_t)r * cols;
        uint16_t* dr = dst + (size_t)r * cols;
        for (int c = 16 * lane; c < cols; c += 1024) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(sr + c);
            u32x4 o0, o1;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                o0[2 * i] = e4m3_h2(v[i] & 0xFFFFu);
                o0[2 * i + 1] = e4m3_h2(v[i] >> 16);
                o1[2 * i] = e4m3_h2(v[i + 2] & 0xFFFFu);
                o1[2 * i + 1] = e4m3_h2(v[i + 2] >> 16);
            }
            *reinterpret_cast<u32x4*>(dr + c) = o0;
            *reinterpret_cast<u32x4*>(dr + c + 8) = o1;
        }
    }
}

// Every computed row r claims a slot of its token's list: list[t][k] = (r, expert) with k from an atomic counter (so
// the slots come in arbitrary order; the combine puts them in row order). Rows whose token lies outside
// [0, tokens) are left out.
__global__ __launch_bounds__(256) void pf_rows_by_token_kernel(PrefillArgs a, const int64_t* row_token, int* cnt,
                                                               int2* list, int tokens) {
    for (int r = blockIdx.x * 256 + threadIdx.x; r < a.P; r += gridDim.x * 256) {
        const int e = a.pe[r];
        if (e < 0) continue;
        const int64_t t = row_token[r];
        if (t < 0 || t >= tokens) continue;
        const int k = atomicAdd(cnt + t, 1);
        if (k < PF_ROWS_PER_TOKEN) list[t * PF_ROWS_PER_TOKEN + k] = make_int2(r, e);
    }
}

// One wave per (token t, 512 columns): the token's rows (at most PF_ROWS_PER_TOKEN) sorted by row index, then
// out[t] += sum over them in that order of ((H(acc * dsc) * r) * svh_d) * w (fp32; deterministic, no atomics); out is
// fp32 or bf16 (then rounded once, after the add). w = w32[r] or the fp16 w16[r].
__global__ __launch_bounds__(256) void pf_combine_rows_kernel(PrefillArgs a, const int* cnt, const int2* list,
                                                              int tokens) {
    __shared__ int2 srt[4][PF_ROWS_PER_TOKEN];
    const int wv = threadIdx.x >> 6;
    const int t = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * 4 + wv));
    if (t >= tokens) return;
    const int lane = threadIdx.x & 63;
    const float hr = HAD_R * fwht_sign(lane);                        // r and the sign fwht128_x16s leaves
    const int nr = min(cnt[t], PF_ROWS_PER_TOKEN);
    int2 ent = make_int2(0x7FFFFFFF, 0);
    if (lane < nr) ent = list[t * PF_ROWS_PER_TOKEN + lane];
    int rank = 0;
    for (int j = 0; j < nr; ++j) rank += __builtin_amdgcn_readlane(ent.x, j) < ent.x;
    if (lane < nr) srt[wv][rank] = ent;
    __builtin_amdgcn_s_waitcnt(0xc07f);                               // lgkmcnt(0): the wave's LDS writes landed
    __builtin_amdgcn_wave_barrier();
    const int col = blockIdx.y * 512 + 128 * (lane >> 4) + 8 * (lane & 15);
    const bool live = blockIdx.y * 512 + 128 * (lane >> 4) < a.K;
    const int colc = live ? col : 0;
    float sum[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < nr; k0 += 8) {
        const int lk = min(k0 + (lane & 7), max(nr - 1, 0));
        const int2 sl = srt[wv][lk];
        const int pl = sl.x, el = sl.y;
        const int okl = (int)(k0 + (lane & 7) < nr);
        const float wl = a.w32 ? a.w32[pl] : (float)u16_as_h(a.w16[pl]);
        const float dl = a.dsc ? a.dsc[pl] : 1.0f;
        const int64_t svl = a.wt.d_svh[el];
        f32x4 raw[8][2];
        u32x4 sv[8];
        bool ok[8];
        float w[8], ds[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int pos = __builtin_amdgcn_readlane(pl, k);
            ok[k] = __builtin_amdgcn_readlane(okl, k) != 0;
            w[k] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), k));
            ds[k] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, dl), k));
            const uint64_t sp = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)svl, k)) |
                                ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(svl >> 32), k) << 32);
            const float* rp = a.contrib + (size_t)pos * a.K + colc;
            raw[k][0] = *reinterpret_cast<const f32x4*>(rp);
            raw[k][1] = *reinterpret_cast<const f32x4*>(rp + 4);
            const uint16_t* svp = reinterpret_cast<const uint16_t*>(sp) + colc;
#pragma unroll
            for (int i = 0; i < 4; ++i) sv[k][i] = *reinterpret_cast<const uint32_t*>(svp + 2 * i);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            float v[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[i] = raw[k][0][i];
                v[4 + i] = raw[k][1][i];
            }
            if (a.dsc) {
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] *= ds[k];
            }
            fwht128_x16s(v, lane);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t s2 = sv[k][i >> 1];
                const float svf = (float)u16_as_h((i & 1) ? s2 >> 16 : s2 & 0xFFFFu);
                if (ok[k]) sum[i] += v[i] * hr * svf * w[k];
            }
        }
    }
    if (!live || nr == 0) return;
    const size_t o = (size_t)t * a.out_stride + col;
    if (a.odt == DT_F32) {
        float* op = reinterpret_cast<float*>(a.out) + o;
#pragma unroll
        for (int i = 0; i < 8; ++i) op[i] = op[i] + sum[i];
    } else {
        uint16_t* op = reinterpret_cast<uint16_t*>(a.out) + o;
#pragma unroll
        for (int i = 0; i < 8; ++i) op[i] = f32_to_bf16(bf16_to_f32(op[i]) + sum[i]);
    }
}

// ------------------------------------------------------------------------------------------------ launchers

static bool g_pf_attr = false;

// Compute units of the current device (the one-launch schedule's grid: one workgroup per CU), cached per device.
static int pf_device_cus() {
    static int cus[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cus[dev] <= 0) {
        int v = 0;
        cus[dev] = (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) ? v
                                                                                                               : 256;
    }
    return cus[dev];
}

int prefill_setup() {
    if (g_pf_attr) return 0;
    const void* ks[4] = {reinterpret_cast<const void*>(pf_gateup_kernel<false>),
                         reinterpret_cast<const void*>(pf_gateup_kernel<true>),
                         reinterpret_cast<const void*>(pf_down_kernel<false>),
                         reinterpret_cast<const void*>(pf_down_kernel<true>)};
    for (const void* k : ks)
        if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)PF_LDS) != hipSuccess) return -1;
    const void* kss[4] = {reinterpret_cast<const void*>(pf_gateup_small_kernel<false>),
                          reinterpret_cast<const void*>(pf_gateup_small_kernel<true>),
                          reinterpret_cast<const void*>(pf_down_small_kernel<false>),
                          reinterpret_cast<const void*>(pf_down_small_kernel<true>)};
    for (const void* k : kss)
        if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)PF_LDS_S) != hipSuccess) return -1;
    const void* ksm[4] = {reinterpret_cast<const void*>(pf_gateup_mid_kernel<false>),
                          reinterpret_cast<const void*>(pf_gateup_mid_kernel<true>),
                          reinterpret_cast<const void*>(pf_down_mid_kernel<false>),
                          reinterpret_cast<const void*>(pf_down_mid_kernel<true>)};
    for (const void* k : ksm)
        if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)PF_LDS_M) != hipSuccess) return -1;
    const void* ksc[3] = {reinterpret_cast<const void*>(pf_sched_kernel<PF_SCHED_E3>),
                          reinterpret_cast<const void*>(pf_sched_kernel<PF_SCHED_E4M3_16>),
                          reinterpret_cast<const void*>(pf_sched_kernel<PF_SCHED_E4M3>)};
    for (const void* k : ksc)
        if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)PF_LDS) != hipSuccess) return -1;
    const void* kscm[3] = {reinterpret_cast<const void*>(pf_sched_part_kernel<PF_SCHED_E3, PF_MID>),
                           reinterpret_cast<const void*>(pf_sched_part_kernel<PF_SCHED_E4M3_16, PF_MID>),
                           reinterpret_cast<const void*>(pf_sched_part_kernel<PF_SCHED_E4M3, PF_MID>)};
    for (const void* k : kscm)
        if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)PF_LDS_M) != hipSuccess) return -1;
    const void* kscs[3] = {reinterpret_cast<const void*>(pf_sched_part_kernel<PF_SCHED_E3, PF_SMALL>),
                           reinterpret_cast<const void*>(pf_sched_part_kernel<PF_SCHED_E4M3_16, PF_SMALL>),
                           reinterpret_cast<const void*>(pf_sched_part_kernel<PF_SCHED_E4M3, PF_SMALL>)};
    for (const void* k : kscs)
        if (hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)PF_LDS_S) != hipSuccess) return -1;
    g_pf_attr = true;
    return 0;
}

// Which grouped GEMMs a call runs. Tiles of few rows are bound by the weight decode on the VALU, and the 256-row
// kernels run one workgroup per CU (160 KB of staging, 256 accumulator registers), which leaves the VALU idle at
// every barrier and load wait. The mid- and small-tile kernels run two workgroups per CU, at the price of decoding
// a segment's weights once per 128-row half or 64-row quarter. Measured at 288 experts, top-8 (E3 numerics /
// trellis-sourced e4m3), against the 256-row kernels:
//   T = 2048 (~57 rows per expert):  mid 27 % faster / small 18 % faster (mid 3 % slower);
//   T = 4096 (~114 rows):            mid 29 % faster / mid 21 % faster (small 3 % slower);
//   T = 6144 (~171 rows):            mid 4 % slower;
//   T = 8192 (~228 rows):            mid 8 % slower, small 47 % slower; Zipf-skewed routing: mid 4 % faster.
// Hence: P <= 64 n: mid (small for e4m3); P <= 128 n: mid; larger calls: the 256-row kernels. "hybrid" splits a
// call by segment size (segments of at most PF_SMALL_ROWS rows on the small tiles, larger ones on the 256-row
// tiles). The environment variable MI355MOE_PREFILL_TILES = "small", "mid", "large" or "hybrid" forces a choice;
// all give bit-identical results (a row's arithmetic does not depend on the tile that holds it).
constexpr int PF_SMALL_ROWS = 128;
enum { PF_TILES_SMALL = 1, PF_TILES_LARGE = 2, PF_TILES_BOTH = 3, PF_TILES_MID = 4 };
static int pf_tiles(const PrefillArgs& a) {
    const char* f = getenv("MI355MOE_PREFILL_TILES");
    if (f && !strcmp(f, "mid")) return PF_TILES_MID;
    if (f && !strcmp(f, "small")) return PF_TILES_SMALL;
    if (f && !strcmp(f, "large")) return PF_TILES_LARGE;
    if (f && !strcmp(f, "hybrid")) return PF_TILES_BOTH;
    if (a.n <= 0) return PF_TILES_LARGE;
    const int64_t P = a.P, n = a.n;
    if (P <= 64 * n) return a.e4m3 ? PF_TILES_SMALL : PF_TILES_MID;
    return P <= 128 * n ? PF_TILES_MID : PF_TILES_LARGE;
}

int launch_prefill(const PrefillArgs& a0, hipStream_t st, int kernels) {
    if (prefill_setup()) return -1;
    PrefillArgs a = a0;
    const bool f8 = a.e4m3 != 0;
    if (f8 && (a.K > 4 * 128 * PF_GATHER_PASSES || !a.asc)) return -1;
    // e4m3 gate/up writes a16out, h2 (down16) or vd + amaxd; the down-input quantization needs vd, amaxd and dsc, the
    // e4m3 down GEMM's combine dsc
    if (f8 && (kernels & 2) && !a.down16 && !a.a16out && (!a.vd || !a.amaxd)) return -1;
    const bool quantd = f8 && !a.down16 && (kernels & 4) && !(kernels & PF_NO_QUANTD);
    if (quantd && (!a.vd || !a.amaxd || !a.dsc)) return -1;
    if (f8 && !a.down16 && (kernels & 8) && !a.dsc) return -1;
    const bool f8dn = f8 && !a.down16;                              // the down GEMM rounds its weights to e4m3
    if (kernels & 1) {
        if (f8) hipLaunchKernelGGL(pf_gather8_kernel, dim3(4096), dim3(256), 0, st, a);
        else hipLaunchKernelGGL(pf_gather_kernel, dim3(4096), dim3(256), 0, st, a);
    }
    const int sg = (a.S_cap + 7) / 8;                               // segment groups of 8 (one per XCD)
    const dim3 gu(8 * (a.N / 128) * sg), dn(8 * (a.K / 256) * sg);
    const int sgs = (4 * a.S_cap + 7) / 8;                          // small tiles: four quarters per segment
    const dim3 gus(8 * (a.N / 128) * sgs), dns(8 * (a.K / 256) * sgs);
    const int sgm = (2 * a.S_cap + 7) / 8;                          // mid tiles: two halves per segment
    const dim3 gum(8 * (a.N / 128) * sgm), dnm(8 * (a.K / 256) * sgm);
    const int tiles = pf_tiles(a0);
    a.small_rows = tiles == PF_TILES_BOTH ? PF_SMALL_ROWS : 0;
    // The one-launch schedule, for calls that run gate/up and down (and, e4m3, the down-input quantisation) on one
    // tile kind: when forced, or by itself, where it measured faster than the separate launches on every tile kind
    // and numerics (288 experts, bit-identical; T = 8192 256-row tiles, uniform routing: E3 -1 to -4 %, DOWN16
    // -1.6 %, e4m3 -1.2 %; Zipf(1.2) routing: E3 -2.1 %, DOWN16 -0.7 %, e4m3 -0.9 %; T = 2048 / 4096 128- and 64-row
    // tiles: E3 0 to -1.7 %, DOWN16 -3.5 %, e4m3 -3.6 / -2.3 %, e4m3 T = 4096 Zipf -4.9 %). MI355MOE_SCHED=separate turns the automatic choice off. (The control words are
    // zeroed by the call's gather or, on row tables, by the row-table setup.)
    const bool sched_ok = (kernels & 6) == 6 && !(kernels & PF_NO_QUANTD) && tiles != PF_TILES_BOTH;
    if (a.sched && a.sched_force && !sched_ok) return -1;
    const char* sched_env = getenv("MI355MOE_SCHED");
    const bool sched_auto = !(sched_env && !strcmp(sched_env, "separate"));
    const bool sched = a.sched && sched_ok && (a.sched_force || sched_auto);
    if (sched) {
        a.small_rows = 0;
        const int parts = tiles == PF_TILES_SMALL ? 4 : tiles == PF_TILES_MID ? 2 : 1;
        const int per_cu = parts > 1 ? 2 : 1;
        const int64_t items = (int64_t)std::max(a.S_cap, 0) * parts * ((a.N >> 7) + (a.K >> 8));
        const dim3 grid((unsigned)std::min<int64_t>((int64_t)per_cu * pf_device_cus(), items)), blk(PF_THREADS);
        const int mode = !f8 ? 0 : a.down16 ? 1 : 2;
        if (grid.x > 0) {
            if (parts == 1) {
                if (mode == 0) hipLaunchKernelGGL(pf_sched_kernel<PF_SCHED_E3>, grid, blk, PF_LDS, st, a);
                else if (mode == 1) hipLaunchKernelGGL(pf_sched_kernel<PF_SCHED_E4M3_16>, grid, blk, PF_LDS, st, a);
                else hipLaunchKernelGGL(pf_sched_kernel<PF_SCHED_E4M3>, grid, blk, PF_LDS, st, a);
            } else if (parts == 2) {
                if (mode == 0) hipLaunchKernelGGL((pf_sched_part_kernel<PF_SCHED_E3, PF_MID>), grid, blk, PF_LDS_M, st, a);
                else if (mode == 1)
                    hipLaunchKernelGGL((pf_sched_part_kernel<PF_SCHED_E4M3_16, PF_MID>), grid, blk, PF_LDS_M, st, a);
                else hipLaunchKernelGGL((pf_sched_part_kernel<PF_SCHED_E4M3, PF_MID>), grid, blk, PF_LDS_M, st, a);
            } else {
                if (mode == 0)
                    hipLaunchKernelGGL((pf_sched_part_kernel<PF_SCHED_E3, PF_SMALL>), grid, blk, PF_LDS_S, st, a);
                else if (mode == 1)
                    hipLaunchKernelGGL((pf_sched_part_kernel<PF_SCHED_E4M3_16, PF_SMALL>), grid, blk, PF_LDS_S, st, a);
                else hipLaunchKernelGGL((pf_sched_part_kernel<PF_SCHED_E4M3, PF_SMALL>), grid, blk, PF_LDS_S, st, a);
            }
        }
        kernels &= ~6;
    }
    if (kernels & 2) {
        if (tiles & PF_TILES_LARGE) {
            if (f8) hipLaunchKernelGGL(pf_gateup_kernel<true>, gu, dim3(PF_THREADS), PF_LDS, st, a);
            else hipLaunchKernelGGL(pf_gateup_kernel<false>, gu, dim3(PF_THREADS), PF_LDS, st, a);
        }
        if (tiles & PF_TILES_SMALL) {
            if (f8) hipLaunchKernelGGL(pf_gateup_small_kernel<true>, gus, dim3(PF_THREADS), PF_LDS_S, st, a);
            else hipLaunchKernelGGL(pf_gateup_small_kernel<false>, gus, dim3(PF_THREADS), PF_LDS_S, st, a);
        }
        if (tiles & PF_TILES_MID) {
            if (f8) hipLaunchKernelGGL(pf_gateup_mid_kernel<true>, gum, dim3(PF_THREADS), PF_LDS_M, st, a);
            else hipLaunchKernelGGL(pf_gateup_mid_kernel<false>, gum, dim3(PF_THREADS), PF_LDS_M, st, a);
        }
    }
    if (kernels & 4) {
        if (quantd) hipLaunchKernelGGL(pf_quantd_kernel, dim3(4096), dim3(256), 0, st, a);
        if (tiles & PF_TILES_LARGE) {
            if (f8dn) hipLaunchKernelGGL(pf_down_kernel<true>, dn, dim3(PF_THREADS), PF_LDS, st, a);
            else hipLaunchKernelGGL(pf_down_kernel<false>, dn, dim3(PF_THREADS), PF_LDS, st, a);
        }
        if (tiles & PF_TILES_SMALL) {
            if (f8dn) hipLaunchKernelGGL(pf_down_small_kernel<true>, dns, dim3(PF_THREADS), PF_LDS_S, st, a);
            else hipLaunchKernelGGL(pf_down_small_kernel<false>, dns, dim3(PF_THREADS), PF_LDS_S, st, a);
        }
        if (tiles & PF_TILES_MID) {
            if (f8dn) hipLaunchKernelGGL(pf_down_mid_kernel<true>, dnm, dim3(PF_THREADS), PF_LDS_M, st, a);
            else hipLaunchKernelGGL(pf_down_mid_kernel<false>, dnm, dim3(PF_THREADS), PF_LDS_M, st, a);
        }
    }
    if (kernels & 8) hipLaunchKernelGGL(pf_combine_kernel, dim3((a.T + 3) / 4, (a.K + 511) / 512), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_zero_out(const PrefillArgs& a, hipStream_t st) {
    const int64_t items = (int64_t)a.T * (a.K / 8);
    if (items > 0)
        hipLaunchKernelGGL(pf_zero_out_kernel, dim3((unsigned)std::max<int64_t>(1, std::min<int64_t>(4096, (items + 255) / 256))),
                           dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_prefill_rows(const PrefillArgs& a0, const RowsPlan& p, hipStream_t st) {
    if (prefill_setup()) return -1;
    if (p.tokens > 0 && (a0.contrib_bf16 || !p.row_token || !p.cnt || !p.list)) return -1;   // fp32 accumulators
    if (p.tok32 && !p.row_token) return -1;
    PrefillArgs a = a0;
    a.pe = p.pe;
    const int fill = std::max(1, std::min(2048, (std::max(a.P, p.tokens) + 255) / 256));
    hipLaunchKernelGGL(pf_rows_init_kernel, dim3(fill), dim3(256), 0, st, a, p.pe, p.cnt, std::max(p.tokens, 0),
                       p.tok32, p.row_token);
    if (a.S_cap > 0) hipLaunchKernelGGL(pf_seg_rows_kernel, dim3(a.S_cap), dim3(256), 0, st, a, p.pe);
    if (p.a8 && p.a8_rows > 0)
        hipLaunchKernelGGL(pf_widen8_kernel, dim3(std::max(1, std::min(4096, (p.a8_rows + 3) / 4))), dim3(256), 0, st,
                           p.a8, p.a8_dst, p.a8_cols, p.a8_rows, p.a8_all ? nullptr : p.pe);
    if (p.kernels)
        if (launch_prefill(a, st, p.kernels)) return -1;
    if (p.tokens > 0) {
        hipLaunchKernelGGL(pf_rows_by_token_kernel, dim3(std::max(1, std::min(2048, (a.P + 255) / 256))), dim3(256), 0,
                           st, a, p.row_token, p.cnt, p.list, p.tokens);
        hipLaunchKernelGGL(pf_combine_rows_kernel, dim3((p.tokens + 3) / 4, (a.K + 511) / 512), dim3(256), 0, st, a,
                           p.cnt, p.list, p.tokens);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace mi355moe
