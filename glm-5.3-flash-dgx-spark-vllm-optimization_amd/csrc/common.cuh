// Shared device helpers for the routed-MoE kernels on gfx950 (CDNA4, wave64).
//
// EXL3 4-bit trellis tiles (code/fork/kernels/exl3_format_ref.py:13-27): a 16x16 tile is 32 little-endian
// 32-bit words; value p of the tile is the 16-bit state s ending at stream bit 4p+4, decoded as
//   x = s * 0xCBAC1FED (mod 2^32); x = (x & 0x8FFF8FFF) ^ 0x3B603B60; v = fp16(x.lo) + fp16(x.hi) (one rounding)
// and placed at row 2(l%4) + (j&1) + 8((j>>1)&1), column l/4 + 8(j>>2) with l = p/8, j = p%8.
//
// Lane mapping used by every decode kernel here: eight consecutive lanes own one tile; lane q (0..7) of the tile
// loads words 4q..4q+3 with one 16-byte load and needs word 4q-1 (held by lane q-1, or by lane 7 of the same
// tile for q = 0). Word 4q+i holds column q and column q+8 at rows 2i, 2i+1, 2i+8, 2i+9, so a lane owns two whole
// columns of the tile (all 16 k rows) and a GEMV needs no cross-lane reduction inside a tile.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace mi355moe {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float HAD_R = 0.088388347648f;   // 1/sqrt(128) as fp32 (ExLlamaV3's r_scale, exl3.cu:37-39)
constexpr uint32_t MCG_MUL = 0xCBAC1FEDu, MCG_MASK = 0x8FFF8FFFu, MCG_FLIP = 0x3B603B60u;

__device__ __forceinline__ _Float16 u16_as_h(uint32_t v) { return __builtin_bit_cast(_Float16, (uint16_t)v); }
__device__ __forceinline__ uint32_t h_as_u16(_Float16 h) { return (uint32_t)__builtin_bit_cast(uint16_t, h); }
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

// fp32 -> bf16 bits, round to nearest even (finite inputs; NaN kept quiet)
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7F800000u) == 0x7F800000u) return (uint16_t)((u >> 16) | ((u & 0xFFFFu) ? 0x40u : 0u));
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// Two fp32 values rounded to bf16 (round to nearest even, gfx950's v_cvt_pk_bf16_f32), packed lo | hi << 16.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const bf16x2_t v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

// The codebook value of one 16-bit state (s < 2^16).
__device__ __forceinline__ _Float16 mcg_value(uint32_t s) {
    const uint32_t x = ((s * MCG_MUL) & MCG_MASK) ^ MCG_FLIP;
    return u16_as_h(x & 0xFFFFu) + u16_as_h(x >> 16);
}

// Decode one trellis word w (its predecessor pw) into the four fp16 pairs of this lane's two columns:
//   d[0] = (k 2i, 2i+1) and d[1] = (k 2i+8, 2i+9) of column q; d[2], d[3] the same rows of column q+8,
// where i = the word's index inside the lane's four words (word 4q+i). State j of the word is
// bits 28-4j .. 43-4j of the 64-bit pair (pw, w).
__device__ __forceinline__ void decode_word(uint32_t pw, uint32_t w, h2 (&d)[4]) {
    const uint32_t D = __builtin_amdgcn_alignbit(pw, w, 20);        // (pw:w) >> 20
    const _Float16 v0 = mcg_value(__builtin_amdgcn_ubfe(D, 8, 16));
    const _Float16 v1 = mcg_value(__builtin_amdgcn_ubfe(D, 4, 16));
    const _Float16 v2 = mcg_value(D & 0xFFFFu);
    const _Float16 v3 = mcg_value(w >> 16);
    const _Float16 v4 = mcg_value(__builtin_amdgcn_ubfe(w, 12, 16));
    const _Float16 v5 = mcg_value(__builtin_amdgcn_ubfe(w, 8, 16));
    const _Float16 v6 = mcg_value(__builtin_amdgcn_ubfe(w, 4, 16));
    const _Float16 v7 = mcg_value(w & 0xFFFFu);
    d[0] = h2{v0, v1};
    d[1] = h2{v2, v3};
    d[2] = h2{v4, v5};
    d[3] = h2{v6, v7};
}

// Word 4q-1 for this lane: lane q-1's last word, or lane 7's of the same tile for q = 0.
__device__ __forceinline__ uint32_t prev_word(uint32_t w3, int lane) {
    return (uint32_t)__shfl((int)w3, (lane & ~7) | ((lane + 7) & 7), 64);
}

// The lane index from an opaque instruction sequence: values derived from it are recomputed where used instead of
// being kept live (or spilled) across a long loop.
__device__ __forceinline__ int opaque_lane() {
    int l;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
    return l;
}

// threadIdx.x through an opaque instruction: the same use-where-defined effect for code that runs once per work item
// inside a persistent loop (values derived from it are not hoisted out of the loop and kept live across items).
__device__ __forceinline__ int opaque_tid() {
    int t;
    asm volatile("v_mov_b32 %0, %1" : "=v"(t) : "v"((int)threadIdx.x));
    return t;
}

// v[i] += c * v[i] of lane l ^ m for the 8 values, one v_fmac_f32 with a DPP source per value (control CTL:
// quad_perm [1,0,3,2] for m = 1, [2,3,0,1] for m = 2, row_ror:8 for m = 8). s_nop 1 gives the two wait states a DPP
// read needs after a VALU write of its source; inside the block each source was written eight instructions earlier.
#define MI355_FMAC_DPP8(v, c, CTL)                                                                                   \
    asm("s_nop 1\n\t"                                                                                             \
        "v_fmac_f32_dpp %0, %0, %8 " CTL " row_mask:0xf bank_mask:0xf\n\t"                                         \
        "v_fmac_f32_dpp %1, %1, %8 " CTL " row_mask:0xf bank_mask:0xf\n\t"                                         \
        "v_fmac_f32_dpp %2, %2, %8 " CTL " row_mask:0xf bank_mask:0xf\n\t"                                         \
        "v_fmac_f32_dpp %3, %3, %8 " CTL " row_mask:0xf bank_mask:0xf\n\t"                                         \
        "v_fmac_f32_dpp %4, %4, %8 " CTL " row_mask:0xf bank_mask:0xf\n\t"                                         \
        "v_fmac_f32_dpp %5, %5, %8 " CTL " row_mask:0xf bank_mask:0xf\n\t"                                         \
        "v_fmac_f32_dpp %6, %6, %8 " CTL " row_mask:0xf bank_mask:0xf\n\t"                                         \
        "v_fmac_f32_dpp %7, %7, %8 " CTL " row_mask:0xf bank_mask:0xf"                                               \
        : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7])        \
        : "v"(c))

// 128-point Walsh-Hadamard of four blocks per wave held 8 consecutive elements per lane (block = lane / 16, elements
// 8 (lane % 16) .. + 7), in the butterfly order of fwht128_w64 (element strides 1, 2, 4 in registers, then 8, 16, 32,
// 64 across lanes xor 1, 2, 4, 8 inside each 16-lane row, by DPP), each value returned times the lane's sign
// fwht_sign(lane) = (-1)^popcount(lane % 16). The butterfly's upper element is a - b; a cross-lane stage here keeps
// own + c * partner with c = -1 on the upper lane of a pair (for lanes xor 1, 2, 8 one v_fmac_f32 with a DPP source
// per value), i.e. the upper result negated. Round-to-nearest is symmetric, so every value is the butterfly's, bit for
// bit, up to that sign; the caller folds the sign into its next multiply (an exact +-1 factor).
__device__ __forceinline__ float fwht_sign(int lane) { return (__builtin_popcount(lane & 15) & 1) ? -1.0f : 1.0f; }
__device__ __forceinline__ void fwht128_x16s(float (&v)[8], int lane) {
#pragma unroll
    for (int h = 1; h < 8; h <<= 1) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (!(i & h)) {
                const float a = v[i], b = v[i + h];
                v[i] = a + b;
                v[i + h] = a - b;
            }
    }
    const float c1 = (lane & 1) ? -1.0f : 1.0f, c2 = (lane & 2) ? -1.0f : 1.0f, c4 = (lane & 4) ? -1.0f : 1.0f,
                c8 = (lane & 8) ? -1.0f : 1.0f;
    MI355_FMAC_DPP8(v, c1, "quad_perm:[1,0,3,2]");
    MI355_FMAC_DPP8(v, c2, "quad_perm:[2,3,0,1]");
#pragma unroll
    for (int i = 0; i < 8; ++i) {                                     // lane ^ 4: row_ror:12 reads lane + 4 (banks 0, 2),
        const int x = __builtin_bit_cast(int, v[i]);                  // row_ror:4 lane - 4 (banks 1, 3)
        const int lo = __builtin_amdgcn_mov_dpp(x, 0x12C, 0xF, 0xF, true);
        const float p = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(lo, x, 0x124, 0xF, 0xA, false));
        v[i] = __builtin_fmaf(p, c4, v[i]);                           // exact product, one rounding
    }
    MI355_FMAC_DPP8(v, c8, "row_ror:8");
}

// NV independent fwht128_x16s, stage by stage: every stage issues its NV x 8 independent operations before the next
// stage reads them, so a single wave per SIMD does not wait on each stage's latency. Each vector's values are those
// of fwht128_x16s, bit for bit (the same operations in the same order per value).
template <int NV>
__device__ __forceinline__ void fwht128_x16s_n(float (&v)[NV][8], int lane) {
#pragma unroll
    for (int h = 1; h < 8; h <<= 1) {
#pragma unroll
        for (int n = 0; n < NV; ++n)
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (!(i & h)) {
                    const float a = v[n][i], b = v[n][i + h];
                    v[n][i] = a + b;
                    v[n][i + h] = a - b;
                }
    }
    const float c1 = (lane & 1) ? -1.0f : 1.0f, c2 = (lane & 2) ? -1.0f : 1.0f, c4 = (lane & 4) ? -1.0f : 1.0f,
                c8 = (lane & 8) ? -1.0f : 1.0f;
#pragma unroll
    for (int n = 0; n < NV; ++n) MI355_FMAC_DPP8(v[n], c1, "quad_perm:[1,0,3,2]");
#pragma unroll
    for (int n = 0; n < NV; ++n) MI355_FMAC_DPP8(v[n], c2, "quad_perm:[2,3,0,1]");
#pragma unroll
    for (int n = 0; n < NV; ++n)
#pragma unroll
        for (int i = 0; i < 8; ++i) {                                 // lane ^ 4, as in fwht128_x16s
            const int x = __builtin_bit_cast(int, v[n][i]);
            const int lo = __builtin_amdgcn_mov_dpp(x, 0x12C, 0xF, 0xF, true);
            const float p = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(lo, x, 0x124, 0xF, 0xA, false));
            v[n][i] = __builtin_fmaf(p, c4, v[n][i]);
        }
#pragma unroll
    for (int n = 0; n < NV; ++n) MI355_FMAC_DPP8(v[n], c8, "row_ror:8");
}

// The value of lane l ^ M (M = 1, 2, 4, 8, 16, 32) without LDS: quad permutes (1, 2), two row rotations with bank
// masks (4), a row rotation (8), v_permlane16_swap (16) and v_permlane32_swap (32).
template <int M>
__device__ __forceinline__ float xor_lane(float v, int lane) {
    const int x = __builtin_bit_cast(int, v);
    if constexpr (M == 1) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, true));
    if constexpr (M == 2) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, true));
    if constexpr (M == 4) {
        const int lo = __builtin_amdgcn_mov_dpp(x, 0x12C, 0xF, 0xF, true);          // row_ror:12: lane + 4
        return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(lo, x, 0x124, 0xF, 0xA, false));  // lane - 4
    }
    if constexpr (M == 8) return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, true));
    if constexpr (M == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap((unsigned)x, (unsigned)x, false, false);
        return __builtin_bit_cast(float, (lane & 16) ? r[0] : r[1]);
    }
    const auto r = __builtin_amdgcn_permlane32_swap((unsigned)x, (unsigned)x, false, false);
    return __builtin_bit_cast(float, (lane & 32) ? r[0] : r[1]);
}

// 128-point Walsh-Hadamard of one row held as two values per lane (lane l: elements 2l, 2l+1) of a wave:
// butterfly strides 1 (in registers), then 2, 4, ..., 64 across lanes xor 1, 2, ..., 32; the lower element of
// every pair keeps a + b, the upper a - b (the fixed fp32 order of exl3.cu:273-284).
__device__ __forceinline__ void fwht128_w64(float& a, float& b, int lane) {
    const float s = a + b, d = a - b;
    a = s;
    b = d;
    auto stage = [&](auto mc) {
        constexpr int m = decltype(mc)::value;
        const float pa = xor_lane<m>(a, lane), pb = xor_lane<m>(b, lane);
        const bool up = (lane & m) != 0;
        a = up ? pa - a : a + pa;
        b = up ? pb - b : b + pb;
    };
    stage(std::integral_constant<int, 1>());
    stage(std::integral_constant<int, 2>());
    stage(std::integral_constant<int, 4>());
    stage(std::integral_constant<int, 8>());
    stage(std::integral_constant<int, 16>());
    stage(std::integral_constant<int, 32>());
}

// 128-point Walsh-Hadamard of a row held as four values per lane by 32 lanes (lane l of the half-wave:
// elements 4l..4l+3); strides 1, 2 in registers, 4..64 across lanes xor 1..16 (same order as above).
__device__ __forceinline__ void fwht128_h32(float (&v)[4], int lane) {
    const float a = v[0] + v[1], b = v[0] - v[1], c = v[2] + v[3], d = v[2] - v[3];
    v[0] = a + c;
    v[1] = b + d;
    v[2] = a - c;
    v[3] = b - d;
#pragma unroll
    for (int m = 1; m < 32; m <<= 1) {
        const bool up = (lane & m) != 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float p = __shfl_xor(v[i], m, 64);
            v[i] = up ? p - v[i] : v[i] + p;
        }
    }
}

// sigmoid as the oracle defines it: 1 / (1 + (float)exp(-(double)g)) with IEEE fp32 division
__device__ __forceinline__ float sigmoid_dexp(float g) {
    const float e = (float)exp(-(double)g);
    return __fdiv_rn(1.0f, 1.0f + e);
}

// sigmoid in fp32 for the wide prefill epilogues (within a few ulp of sigmoid_dexp): e^-g = 2^y (1 + e ln 2) with
// y = fp32(-g log2 e) and e its rounding residual, then one reciprocal (v_exp_f32 and v_rcp_f32 are ~1 ulp each)
__device__ __forceinline__ float sigmoid_fast(float g) {
    constexpr float L2E = 1.44269502162933349609375f, L2E_LO = 1.925963033500011079e-8f, LN2 = 0.693147180559945f;
    const float y = -g * L2E;
    const float e = __builtin_fmaf(-g, L2E, -y) - g * L2E_LO;
    const float t = __builtin_amdgcn_exp2f(y);
    return __builtin_amdgcn_rcpf(1.0f + __builtin_fmaf(t, e * LN2, t));
}

// Split-K partials cross workgroups (and XCDs, each with its own L2) through device-coherent accesses instead of
// L2 write-back / invalidate fences: partials are stored and re-loaded as relaxed agent-scope atomics (stores write
// through to the device coherence point, loads do not hit stale lines), and the arrival counter is bumped only
// after every store of the workgroup has completed (s_waitcnt + barrier).
__device__ __forceinline__ void st_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coherent(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent(int* p, int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int ld_coherent(const int* p) {
    return __hip_atomic_load(const_cast<int*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------------------------- LDS staging

// Wave instruction: 64 lanes x 16 bytes, lane l -> LDS bytes lds_wave + 16 l (global_load_lds_dwordx4). Written as
// inline assembly so the compiler adds no wait of its own for these loads: the kernels wait for them explicitly
// (WAIT_VM) before the barrier that publishes a stage, and issue no other global loads while any are in flight.
__device__ __forceinline__ void dma16(const void* src_lane, unsigned char* lds_wave) {
    const uint32_t m0 = (uint32_t)(uintptr_t)lds_wave;
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(m0), "v"(src_lane)
                 : "memory", "m0");
}
// The same marked non-temporal (data read once, e.g. streamed weights).
__device__ __forceinline__ void dma16_nt(const void* src_lane, unsigned char* lds_wave) {
    const uint32_t m0 = (uint32_t)(uintptr_t)lds_wave;
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off nt" ::"s"(m0), "v"(src_lane)
                 : "memory", "m0");
}
// The same as a device-coherent load (agent scope, sc1: the data comes from the device coherence point, not from a
// line another XCD's stores left stale in this CU's or XCD's caches).
__device__ __forceinline__ void dma16_coh(const void* src_lane, unsigned char* lds_wave) {
    const uint32_t m0 = (uint32_t)(uintptr_t)lds_wave;
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off sc1" ::"s"(m0), "v"(src_lane)
                 : "memory", "m0");
}
// Device-coherent 16-byte accesses (sc1: agent scope, served by the device coherence point, the cache policy
// agent-scope relaxed atomics take) through a buffer resource over a wave-uniform base address: one instruction
// where an atomic access moves at most 8 bytes. Offsets are in bytes from the base, below 2^31.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t coh_rsrc(const void* base) {
    const uint64_t p = (uint64_t)(uintptr_t)base;
    const uint64_t u = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)p) |
                       ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(p >> 32)) << 32);
    return __builtin_amdgcn_make_buffer_rsrc((void*)(uintptr_t)u, (short)0, 0x7FFFFFFF, 0x00020000);
}
constexpr int COH_SC1 = 16;                       // the buffer instructions' cache-policy bit for sc1
__device__ __forceinline__ u32x4 ld_coh16(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, COH_SC1));
}
__device__ __forceinline__ void st_coh16(__amdgpu_buffer_rsrc_t r, int off, u32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, COH_SC1);
}
// The same with 4 bytes per lane: lane l -> LDS bytes lds_wave + 4 l (global_load_lds_dword).
__device__ __forceinline__ void dma4(const void* src_lane, unsigned char* lds_wave) {
    const uint32_t m0 = (uint32_t)(uintptr_t)lds_wave;
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off" ::"s"(m0), "v"(src_lane)
                 : "memory", "m0");
}

// s_waitcnt vmcnt(n) lgkmcnt(0) (n <= 63; vmcnt bits 3:0 and 15:14): this wave's staged loads up to the one n before
// the last have landed in LDS, and its LDS reads of the buffer about to be refilled have returned
#define WAIT_VM(n) __builtin_amdgcn_s_waitcnt(0x0070 | ((n) & 15) | (((n) >> 4) << 14))
#define LDS_BARRIER() asm volatile("s_barrier" ::: "memory")

}  // namespace mi355moe
