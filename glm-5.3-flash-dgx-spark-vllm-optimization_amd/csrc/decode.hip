// Decode-path kernels (few rows per expert): trellis dequant, input rotation, the grouped gate/up and down trellis
// GEMVs with their epilogues fused through split-K arrival counters, and the slot-order combine.
//
// Work decomposition of the grouped GEMVs (a few rows per expert: the work is a stream of 4-bit codes):
//   workgroup (128-column block cb, K split ks, row segment s) of 4 waves; wave w owns 32 columns over the split's
//   K range and steps through it four k tiles at a time. Each lane loads 16 bytes of trellis per step and matrix
//   (a quarter of one 16x16 tile), decodes its 32 states to raw codebook words, and hands each word's (lo, hi)
//   fp16 halves to v_mfma_f32_16x16x32_f16 as the B operand, with the rows' inputs duplicated per k as the A
//   operand (staged in LDS in that order). The matrix core therefore performs the codebook's lo + hi sum and the
//   dot product for up to 16 rows at once; the VALU only extracts states, multiplies and masks. Each split stores
//   its fp32 partial; the workgroup that arrives last for (s, cb) adds the splits in split order and runs the
//   epilogue, so every result is independent of scheduling.
// Numerics (oracle/csrc/oracle.c mode 4 = mode 0 with unrounded codebook sums):
//   rot_in   xg = fp16(H(fp16(x * suh_g)) * r)                       (exl3.cu:321-349)
//   GEMV     z = sum_k xg[k] * (fp16(lo) + fp16(hi)) in fp32 (the reference rounds lo + hi to fp16 first)
//   gate/up  g = H(sum_k xg Wq_g) * r * svh_g, u likewise (fp32); s = silu(g); s = min(s, L), u = clamp(u, -L, L)
//            iff L != 0 (exl3_moe's order, xl_hadamard_inner.cuh:280-400); a16 = fp16(s*u); xd = fp16(H(fp16(a16 *
//            suh_d)) * r)
//   down     v = H(sum_n xd Wq_d) * (r * w16) * svh_d                   (exl3.cu:455-496)
//   combine  out[t] = sum over the token's slots in slot order (exl3.cu:815-864), or fp32 atomics (accumulate mode)
#include "common.cuh"
#include "mi355moe_internal.h"

namespace mi355moe {

constexpr int DEC_WAVES = 4;

// ------------------------------------------------------------------------------------------------ dequant

// grid (nt / 8, kt), one wave: the eight tiles nt0..nt0+7 of k-tile row a. Writes W_q fp16 [kt*16][nt*16].
__global__ __launch_bounds__(64) void dequant_kernel(const u32x4* __restrict__ tr, int nt, uint16_t* __restrict__ wq) {
    const int lane = threadIdx.x;
    const int t = lane >> 3, q = lane & 7;
    const int a = blockIdx.y, b = blockIdx.x * 8 + t;
    const u32x4 w = tr[((size_t)a * nt + b) * 8 + q];
    const uint32_t pw0 = prev_word(w[3], lane);
    const int ncol = nt * 16;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h2 d[4];
        decode_word(i ? w[i - 1] : pw0, w[i], d);
        const int r0 = a * 16 + 2 * i;
        const int c0 = b * 16 + q;
        uint16_t* o = wq + (size_t)r0 * ncol + c0;
        o[0] = (uint16_t)h_as_u16(d[0].x);
        o[ncol] = (uint16_t)h_as_u16(d[0].y);
        o[8 * ncol] = (uint16_t)h_as_u16(d[1].x);
        o[9 * ncol] = (uint16_t)h_as_u16(d[1].y);
        o[8] = (uint16_t)h_as_u16(d[2].x);
        o[ncol + 8] = (uint16_t)h_as_u16(d[2].y);
        o[8 * ncol + 8] = (uint16_t)h_as_u16(d[3].x);
        o[9 * ncol + 8] = (uint16_t)h_as_u16(d[3].y);
    }
}

// ------------------------------------------------------------------------------------------------ activations

// One input value as fp16: fp16 as stored, bf16 rounded to fp16 (x.half()).
__device__ __forceinline__ void load_x2(const void* x, int xdt, size_t off, _Float16& h0, _Float16& h1) {
    if (xdt == DT_BF16) {
        const uint32_t v = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint16_t*>(x) + off);
        h0 = (_Float16)__builtin_bit_cast(float, v << 16);
        h1 = (_Float16)__builtin_bit_cast(float, v & 0xFFFF0000u);
    } else {
        const h2 v = *reinterpret_cast<const h2*>(reinterpret_cast<const uint16_t*>(x) + off);
        h0 = v.x;
        h1 = v.y;
    }
}

// 128 rotated inputs of one row by one wave: dst[2l], dst[2l+1] = fp16(H(fp16(x * suh)) * r)
__device__ __forceinline__ void rot_in_block(const void* x, int xdt, size_t xoff, const _Float16* suh, _Float16* dst,
                                             int lane) {
    _Float16 h0, h1;
    load_x2(x, xdt, xoff + 2 * lane, h0, h1);
    const h2 s = *reinterpret_cast<const h2*>(suh + 2 * lane);
    float p0 = (float)(_Float16)(h0 * s.x), p1 = (float)(_Float16)(h1 * s.y);
    fwht128_w64(p0, p1, lane);
    *reinterpret_cast<h2*>(dst + 2 * lane) = h2{(_Float16)(p0 * HAD_R), (_Float16)(p1 * HAD_R)};
}

// grid (P, K/128), one wave: out[pos][blk] = rot_in of x[tok[pos]] with expert pe[pos]'s suh; rows with pe < 0 are
// left untouched.
__global__ __launch_bounds__(64) void rot_in_kernel(const void* __restrict__ x, int xdt, int64_t x_stride,
                                                    const int* __restrict__ tok, const int* __restrict__ pe,
                                                    const int64_t* __restrict__ suh_tab, int K,
                                                    uint16_t* __restrict__ out) {
    const int pos = blockIdx.x, blk = blockIdx.y;
    const int e = pe[pos];
    if (e < 0) return;
    const _Float16* suh = reinterpret_cast<const _Float16*>(suh_tab[e]) + blk * 128;
    rot_in_block(x, xdt, (size_t)tok[pos] * x_stride + blk * 128, suh,
                 reinterpret_cast<_Float16*>(out) + (size_t)pos * K + blk * 128, threadIdx.x);
}

// ------------------------------------------------------------------------------------------------ grouped GEMV

// Staged GEMV inputs in LDS (fp16), in the matrix-core operand order: a row holds its k range as 16-half groups per
// k tile, half 4i + m of a group = k 2i + (m & 1) + 8 (m >> 1) of the tile. Word i of a trellis tile holds exactly
// those four k rows (per column), so halves 4i..4i+3, each duplicated into both halves of a dword, form the A
// operand that matches the decoded word. Rows are padded by XPAD halves against bank conflicts.
constexpr int XPAD = 8;
__device__ __forceinline__ int xa_pos(int k) {
    const int kk = k & 15;
    return 16 * (k >> 4) + 4 * ((kk & 7) >> 1) + (kk & 1) + 2 * (kk >> 3);
}

// Staged-input preparation, four 128-blocks per wave (one per 16-lane row, 8 consecutive inputs per lane):
// rot8_load fetches a lane's 8 inputs and 8 suh values, rot8_scale forms fp16(x * suh) as floats (bf16 inputs are
// first rounded to fp16, as x.half() does), fwht128_x16s rotates, and the stores write fp16(v * r) into the staged
// row in the matrix-core order (xa_pos), plain or duplicated.
struct RotIn8 {
    uint32_t x[4];
    u32x4 s;
};
// global-address-space loads (a plain pointer from a pointer table would otherwise become a flat load, which also
// counts against the scalar-load counter and serialises the prologue)
typedef __attribute__((address_space(1))) const uint32_t gu32;
typedef __attribute__((address_space(1))) const u32x4 gu32x4;
__device__ __forceinline__ uint32_t ld_g32(const void* p) {
    return *reinterpret_cast<gu32*>(reinterpret_cast<uintptr_t>(p));
}
__device__ __forceinline__ u32x4 ld_g128(const void* p) {
    return *reinterpret_cast<gu32x4*>(reinterpret_cast<uintptr_t>(p));
}
// x: 4-byte aligned (even row stride), read as dwords; suh: whole 16-byte chunks
__device__ __forceinline__ RotIn8 rot8_load(const void* x, size_t xoff, const _Float16* suh) {
    const uint16_t* xp = reinterpret_cast<const uint16_t*>(x) + xoff;
    return RotIn8{{ld_g32(xp), ld_g32(xp + 2), ld_g32(xp + 4), ld_g32(xp + 6)}, ld_g128(suh)};
}
// branch-free in the input type, so the first use of a load batch needs no control-flow join
__device__ __forceinline__ void rot8_scale(const RotIn8& v, int xdt, float (&p)[8]) {
    const bool bf = xdt == DT_BF16;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t w = v.x[i];
        const _Float16 h0 = bf ? (_Float16)__builtin_bit_cast(float, w << 16) : u16_as_h(w & 0xFFFFu);
        const _Float16 h1 = bf ? (_Float16)__builtin_bit_cast(float, w & 0xFFFF0000u) : u16_as_h(w >> 16);
        // (the suh word goes through a scalar first: hipcc miscompiles bit_cast of an ext_vector element indexed in
        // an unrolled loop, reading element 0 every time)
        const uint32_t sw = v.s[i];
        p[2 * i] = (float)(_Float16)(h0 * u16_as_h(sw & 0xFFFFu));
        p[2 * i + 1] = (float)(_Float16)(h1 * u16_as_h(sw >> 16));
    }
}
__device__ __forceinline__ uint32_t dup16(_Float16 h) {
    const uint32_t u = h_as_u16(h);
    return u | (u << 16);
}
// 8 consecutive values at local k0 (a multiple of 8) of a staged row: value j goes to position xa_pos(k0 + j) =
// 16 (k0 / 16) + 4 (j / 2) + j % 2 + 2 ((k0 / 8) % 2), as halves (plain) or duplicated dwords
__device__ __forceinline__ void stage8_store(const float (&p)[8], float hr, uint16_t* row, int k0) {
    uint16_t* d = row + (k0 & ~15) + 2 * ((k0 >> 3) & 1);
#pragma unroll
    for (int m = 0; m < 4; ++m)
        *reinterpret_cast<h2*>(d + 4 * m) = h2{(_Float16)(p[2 * m] * hr), (_Float16)(p[2 * m + 1] * hr)};
}
__device__ __forceinline__ void stage8_store_dup(const float (&p)[8], float hr, uint32_t* row, int k0) {
    uint32_t* d = row + (k0 & ~15) + 2 * ((k0 >> 3) & 1);
#pragma unroll
    for (int m = 0; m < 4; ++m)
        *reinterpret_cast<uint2*>(d + 4 * m) =
            make_uint2(dup16((_Float16)(p[2 * m] * hr)), dup16((_Float16)(p[2 * m + 1] * hr)));
}

// Segments of up to DUP_ROWS rows stage each input duplicated into a dword (x, x) at dword xa_pos(k) of the row,
// so the matrix-core A operand of a word is one 16-byte LDS read (no per-step permutes).
constexpr int DUP_ROWS = 4;

// The raw codebook word of a state: its two fp16 halves sum to the weight.
__device__ __forceinline__ uint32_t mcg_word(uint32_t s) { return ((s * MCG_MUL) & MCG_MASK) ^ MCG_FLIP; }

// Decode trellis word w (predecessor pw) into matrix-core B operands: b0 = column q, b1 = column q + 8, dword m
// holding the (lo, hi) halves of k row 2i + (m & 1) + 8 (m >> 1) (i = the word's index in the lane's four).
__device__ __forceinline__ void decode_word_b(uint32_t pw, uint32_t w, u32x4& b0, u32x4& b1) {
    const uint32_t D = __builtin_amdgcn_alignbit(pw, w, 20);        // (pw:w) >> 20
    b0[0] = mcg_word(__builtin_amdgcn_ubfe(D, 8, 16));
    b0[1] = mcg_word(__builtin_amdgcn_ubfe(D, 4, 16));
    b0[2] = mcg_word(D & 0xFFFFu);
    b0[3] = mcg_word(w >> 16);
    b1[0] = mcg_word(__builtin_amdgcn_ubfe(w, 12, 16));
    b1[1] = mcg_word(__builtin_amdgcn_ubfe(w, 8, 16));
    b1[2] = mcg_word(__builtin_amdgcn_ubfe(w, 4, 16));
    b1[3] = mcg_word(w & 0xFFFFu);
}

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ f32x4 mfma16(const u32x4& a, const u32x4& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, a), __builtin_bit_cast(h8, b), c, 0, 0, 0);
}

// A operand of word i: staged halves 4i..4i+3 (dwords 2i, 2i + 1 of the step's eight), each duplicated.
__device__ __forceinline__ u32x4 a_operand(const u32x4& x0, const u32x4& x1, int i) {
    const uint32_t d0 = i < 2 ? x0[2 * i] : x1[2 * i - 4], d1 = i < 2 ? x0[2 * i + 1] : x1[2 * i - 3];
    return u32x4{__builtin_amdgcn_perm(d0, d0, 0x01000100u), __builtin_amdgcn_perm(d0, d0, 0x03020302u),
                 __builtin_amdgcn_perm(d1, d1, 0x01000100u), __builtin_amdgcn_perm(d1, d1, 0x03020302u)};
}

// One step of a wave over one matrix: lane (t, q) holds words 4q..4q+3 of the tile (pw0 = word 4q - 1) (k tile t/2 of the step, column
// tile t%2); for word i the matrix core takes A = the rows' staged inputs of that word's four k rows (lane group
// t/2 = lane/16 supplies k tile t/2) and B = the decoded halves of column q (acc[0]) or q + 8 (acc[1]): the MFMA
// adds lo and hi exactly in fp32 together with the products.
__device__ __forceinline__ void step_mfma(const u32x4& w, uint32_t pw0, const u32x4& x0, const u32x4& x1,
                                          f32x4 (&acc)[2]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const u32x4 av = a_operand(x0, x1, i);
        u32x4 b0, b1;
        decode_word_b(i ? w[i - 1] : pw0, w[i], b0, b1);
        acc[0] = mfma16(av, b0, acc[0]);
        acc[1] = mfma16(av, b1, acc[1]);
    }
}

// The same step for gate and up with one shared staged input (one A operand per word for both matrices).
__device__ __forceinline__ void step_mfma2(const u32x4& wg, uint32_t pwg, const u32x4& wu, uint32_t pwu,
                                           const u32x4& x0, const u32x4& x1, f32x4 (&ag)[2], f32x4 (&au)[2]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const u32x4 av = a_operand(x0, x1, i);
        u32x4 b0, b1;
        decode_word_b(i ? wg[i - 1] : pwg, wg[i], b0, b1);
        ag[0] = mfma16(av, b0, ag[0]);
        ag[1] = mfma16(av, b1, ag[1]);
        decode_word_b(i ? wu[i - 1] : pwu, wu[i], b0, b1);
        au[0] = mfma16(av, b0, au[0]);
        au[1] = mfma16(av, b1, au[1]);
    }
}

// step_mfma2 with the A operands read ready-made from a duplicated staged row (xa[i] = word i's).
__device__ __forceinline__ void step_mfma2_dup(const u32x4& wg, uint32_t pwg, const u32x4& wu, uint32_t pwu,
                                               const u32x4 (&xa)[4], f32x4 (&ag)[2], f32x4 (&au)[2]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        u32x4 b0, b1;
        decode_word_b(i ? wg[i - 1] : pwg, wg[i], b0, b1);
        ag[0] = mfma16(xa[i], b0, ag[0]);
        ag[1] = mfma16(xa[i], b1, ag[1]);
        decode_word_b(i ? wu[i - 1] : pwu, wu[i], b0, b1);
        au[0] = mfma16(xa[i], b0, au[0]);
        au[1] = mfma16(xa[i], b1, au[1]);
    }
}

// Issue priority by progress through the K loop: 3 in the first quarter of the steps, down to 0 in the last (the
// loops run as four quarters, so no branch sits inside the step loop). The arbiter favours a CU's oldest waves, so
// the waves of a workgroup drift apart (its last wave finishing ~13 µs after its first at T = 8) and the last ones
// then run with few others to hide their latency; waves behind now issue first, so a workgroup's waves finish
// closer together.
__device__ __forceinline__ void prio_for_quarter(int q) {
    if (q == 0) __builtin_amdgcn_s_setprio(3);
    else if (q == 1) __builtin_amdgcn_s_setprio(2);
    else if (q == 2) __builtin_amdgcn_s_setprio(1);
    else __builtin_amdgcn_s_setprio(0);
}
// The end of quarter q of a loop of `steps` steps taken DEPTH at a time.
template <int DEPTH>
__device__ __forceinline__ int quarter_end(int q, int steps) {
    return q == 3 ? steps : ((q + 1) * steps / 4) / DEPTH * DEPTH;
}

// Streamed weight load: a global-address-space 16-byte load marked non-temporal (read once per call).
__device__ __forceinline__ u32x4 ld_stream(const u32x4* p) {
    return __builtin_nontemporal_load(reinterpret_cast<gu32x4*>(reinterpret_cast<uintptr_t>(p)));
}

// Accumulator layout of a wave (two 16x16 tiles): lane column c = lane % 16 is output column (c/8)*16 + c%8 (acc[0])
// and that + 8 (acc[1]) of the wave's 32; rows 4 (lane/16) + r.
__device__ __forceinline__ int acc_col(int lane) { return ((lane & 15) >> 3) * 16 + (lane & 7); }

constexpr int GU_WAVES = 8;      // gate/up workgroup: 4 column groups of 32 x 2 halves of the K range
constexpr int DN_WAVES = 8;      // down workgroup: 8 column groups of 32 (256 output columns) over the N range
constexpr int ZS_ROWS = 16;

// Arrival of a tile fragment of `len` chunks whose partial sums went to slot `slot`: one 64-bit atomic adds len to
// the tile's chunk count (bits 0-31) and the slot's bit (bits 32-63). Returns true in the workgroup whose fragment
// completes the tile's `total` chunks, with *mask = the slots of every fragment (every fragment's device-coherent
// stores completed before it arrived, and the elected workgroup loads them device-coherent, so no fence is needed).
__device__ __forceinline__ bool arrive_fragment(unsigned long long* c, unsigned len, int slot, unsigned total,
                                                unsigned* mask, int* flag) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned long long add = (unsigned long long)len | (1ull << (32 + slot));
        const unsigned long long now =
            __hip_atomic_fetch_add(c, add, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + add;
        *flag = (unsigned)now == total;
        *mask = (unsigned)(now >> 32);
    }
    __syncthreads();
    return *flag != 0;
}

// 512 threads: workgroup = 128 gate and up columns of one segment over one K range [kc0, kc1) in chunks of kch_gu;
// wave (cg, kh) = columns 32cg..32cg+31 over half kh of the range, DEPTH steps of loads in flight. The halves are
// added in LDS; a fragment covering all of K runs the epilogue directly, otherwise it stores its partial in slot
// `slot` and the fragment that completes the tile adds the slots in order. smem: the dynamic LDS.
template <int DEPTH, bool SHARED>
__device__ __forceinline__ void gateup_tile(const DecodeArgs& a, int cb, int s, int kc0, int kc1, int slot,
                                            unsigned char* smem) {
    __shared__ int last_flag;
    __shared__ unsigned slot_mask;
    if (s >= a.nseg[0]) return;
    const int e = a.seg_expert[s], row0 = a.seg_row0[s], rn = a.seg_rows[s];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int cg = wv & 3, kh = wv >> 2;
    const int K = a.K, N = a.N, NT = N >> 4;
    const int KR = (kc1 - kc0) * a.kch_gu, KH = KR >> 1, kbase = kc0 * a.kch_gu, RSH = KR + XPAD;
    const int KC = K / a.kch_gu;
    constexpr int NMAT = SHARED ? 1 : 2;
    uint16_t* xs = reinterpret_cast<uint16_t*>(smem);              // [NMAT][rn][RSH] halves, or
    uint32_t* xw = reinterpret_cast<uint32_t*>(smem);              // [rn][RSD] duplicated (SHARED, rn <= DUP_ROWS)
    const int RSD = KR + 4;
    const bool dup = SHARED && rn <= DUP_ROWS;

    // prologue: the segment's rotated inputs for this K range as (row, matrix, 128-block) tasks, four per wave at
    // a time (one per 16-lane row), one quad per wave per batch. The first batch's loads are issued unconditionally
    // (task index clamped) before the weight prefetch: loads return in issue order, so inputs queued behind the
    // prefetch would wait for all of it. The segment's token ids are read once, one per lane.
    const int g4 = lane >> 4, l16 = lane & 15;
    const int nb = KR >> 7, ntask = rn * NMAT * nb;
    const int tokl = a.tok[row0 + min(lane, rn - 1)];
    const _Float16* suhg = reinterpret_cast<const _Float16*>(a.wt.g_suh[e]) + kbase;
    const _Float16* suhu = reinterpret_cast<const _Float16*>(a.wt.u_suh[e]) + kbase;
    auto task_of = [&](int c, int t0) { return t0 + 4 * (c * GU_WAVES + wv) + g4; };   // t0: batch base
    auto task_load = [&](int task) {
        task = min(task, ntask - 1);
        const int r = task / (NMAT * nb), rem = task - r * NMAT * nb, mat = rem / nb, b = rem - mat * nb;
        const int tk = __shfl(tokl, r, 64);
        return rot8_load(a.x, (size_t)tk * a.x_stride + kbase + b * 128 + 8 * l16,
                         (mat ? suhu : suhg) + b * 128 + 8 * l16);
    };
    auto task_store = [&](int task, const RotIn8& vv) {
        float p[8];
        rot8_scale(vv, a.xdt, p);
        fwht128_x16s(p, lane);
        const float hr = HAD_R * fwht_sign(lane);                    // r and the sign fwht128_x16s leaves
        const int r = task / (NMAT * nb), rem = task - r * NMAT * nb, mat = rem / nb, b = rem - mat * nb;
        if (task < ntask) {
            if (dup) stage8_store_dup(p, hr, xw + (size_t)r * RSD, b * 128 + 8 * l16);
            else stage8_store(p, hr, xs + (size_t)(mat * rn + r) * RSH, b * 128 + 8 * l16);
        }
    };
    constexpr int QB = 1;                                            // quads per wave per batch
    constexpr int BT = 4 * QB * GU_WAVES;                            // tasks per batch
    RotIn8 v[QB];
#pragma unroll
    for (int c = 0; c < QB; ++c) v[c] = task_load(task_of(c, 0));
    __builtin_amdgcn_sched_barrier(0);

    const int t = lane >> 3, q = lane & 7;
    const int ct = cb * 8 + cg * 2 + (t & 1);
    const u32x4* G = reinterpret_cast<const u32x4*>(a.wt.g_tr[e]);
    const u32x4* U = reinterpret_cast<const u32x4*>(a.wt.u_tr[e]);
    const size_t sstr = (size_t)NT * 8 * 4;                         // one step = four k tiles
    const size_t idx0 = ((size_t)(((kbase + kh * KH) >> 4) + (t >> 1)) * NT + ct) * 8 + q;
    const int steps = KH >> 6;                                       // a multiple of DEPTH
    // buffer j is refilled right after use with step st + DEPTH + j; refills past the last step re-read the last
    // step, so every load is unconditional and in bounds
    u32x4 gb[DEPTH], ub[DEPTH];
#pragma unroll
    for (int j = 0; j < DEPTH; ++j) {
        gb[j] = ld_stream(G + idx0 + j * sstr);
        ub[j] = ld_stream(U + idx0 + j * sstr);
    }
    __builtin_amdgcn_sched_barrier(0);

    // the first batch in straight-line code (so its wait leaves the prefetch in flight), then any further batches
#pragma unroll
    for (int c = 0; c < QB; ++c) task_store(task_of(c, 0), v[c]);
    for (int t0 = BT; t0 < ntask; t0 += BT) {
#pragma unroll
        for (int c = 0; c < QB; ++c) v[c] = task_load(task_of(c, t0));
#pragma unroll
        for (int c = 0; c < QB; ++c) task_store(task_of(c, t0), v[c]);
    }
    __syncthreads();

    const int arow = min(lane & 15, rn - 1);                         // rows >= rn repeat the last row (dropped)
    f32x4 ag[2], au[2];
    ag[0] = ag[1] = au[0] = au[1] = f32x4{0.f, 0.f, 0.f, 0.f};
    // staged inputs are read one step ahead (this step's, the next step's), and so are the predecessor words (pg,
    // pu), so no step waits on its own LDS reads
    uint32_t pg = prev_word(gb[0][3], lane), pu = prev_word(ub[0][3], lane);
    if (dup) {
        const uint32_t* xr = xw + (size_t)arow * RSD + kh * KH + (t >> 1) * 16;
        u32x4 xa[4], xn[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) xa[i] = reinterpret_cast<const u32x4*>(xr)[i];
        for (int q = 0, st = 0; q < 4; ++q) {
          prio_for_quarter(q);
          for (const int st1 = quarter_end<DEPTH>(q, steps); st < st1; st += DEPTH) {
#pragma unroll
            for (int j = 0; j < DEPTH; ++j) {
                const size_t nx = idx0 + (size_t)min(st + DEPTH + j, steps - 1) * sstr;
                const int sn = min(st + j + 1, steps - 1);
                const int jn = (j + 1) % DEPTH;
                const uint32_t pgn = prev_word(gb[jn][3], lane), pun = prev_word(ub[jn][3], lane);
#pragma unroll
                for (int i = 0; i < 4; ++i) xn[i] = reinterpret_cast<const u32x4*>(xr + sn * 64)[i];
                step_mfma2_dup(gb[j], pg, ub[j], pu, xa, ag, au);
                gb[j] = ld_stream(G + nx);
                ub[j] = ld_stream(U + nx);
                __builtin_amdgcn_sched_barrier(0);                  // keep the refill here, not sunk to the end
#pragma unroll
                for (int i = 0; i < 4; ++i) xa[i] = xn[i];
                pg = pgn;
                pu = pun;
            }
          }
        }
    } else {
        const uint16_t* xg = xs + (size_t)arow * RSH + kh * KH + (t >> 1) * 16;
        const uint16_t* xu = xs + (size_t)((NMAT - 1) * rn + arow) * RSH + kh * KH + (t >> 1) * 16;
        u32x4 xc[2][2], xn[2][2];
        xc[0][0] = reinterpret_cast<const u32x4*>(xg)[0];
        xc[0][1] = reinterpret_cast<const u32x4*>(xg)[1];
        if (!SHARED) {
            xc[1][0] = reinterpret_cast<const u32x4*>(xu)[0];
            xc[1][1] = reinterpret_cast<const u32x4*>(xu)[1];
        }
        for (int q = 0, st = 0; q < 4; ++q) {
          prio_for_quarter(q);
          for (const int st1 = quarter_end<DEPTH>(q, steps); st < st1; st += DEPTH) {
#pragma unroll
            for (int j = 0; j < DEPTH; ++j) {
                const size_t nx = idx0 + (size_t)min(st + DEPTH + j, steps - 1) * sstr;
                const int sn = min(st + j + 1, steps - 1);
                const int jn = (j + 1) % DEPTH;
                const uint32_t pgn = prev_word(gb[jn][3], lane), pun = prev_word(ub[jn][3], lane);
                xn[0][0] = reinterpret_cast<const u32x4*>(xg + sn * 64)[0];
                xn[0][1] = reinterpret_cast<const u32x4*>(xg + sn * 64)[1];
                if (SHARED) {
                    step_mfma2(gb[j], pg, ub[j], pu, xc[0][0], xc[0][1], ag, au);
                } else {
                    xn[1][0] = reinterpret_cast<const u32x4*>(xu + sn * 64)[0];
                    xn[1][1] = reinterpret_cast<const u32x4*>(xu + sn * 64)[1];
                    step_mfma(gb[j], pg, xc[0][0], xc[0][1], ag);
                    step_mfma(ub[j], pu, xc[1][0], xc[1][1], au);
                }
                gb[j] = ld_stream(G + nx);
                ub[j] = ld_stream(U + nx);
                __builtin_amdgcn_sched_barrier(0);                  // keep the refill here, not sunk to the end
                xc[0][0] = xn[0][0];
                xc[0][1] = xn[0][1];
                if (!SHARED) {
                    xc[1][0] = xn[1][0];
                    xc[1][1] = xn[1][1];
                }
                pg = pgn;
                pu = pun;
            }
          }
        }
    }

    __builtin_amdgcn_s_setprio(0);
    // the epilogue's column scales (waves with rows to finish) are loaded here, so their latency overlaps the
    // exchange of the K halves and any split-K reduction below (with DEPTH 2 -- short K ranges -- where they are
    // used: there the registers they would hold are the loop's)
    u32x4 svg = {}, svu = {}, sud = {};
    auto load_scales = [&]() {
        const int colb = cb * 128 + 8 * (opaque_lane() & 15);
        svg = ld_g128(reinterpret_cast<const _Float16*>(a.wt.g_svh[e]) + colb);
        svu = ld_g128(reinterpret_cast<const _Float16*>(a.wt.u_svh[e]) + colb);
        sud = ld_g128(reinterpret_cast<const _Float16*>(a.wt.d_suh[e]) + colb);
    };
    if (DEPTH == 4 && wv * 4 < rn) load_scales();
    // the two K halves: kh = 1 hands its accumulators to kh = 0 through LDS, which writes the row sums
    __syncthreads();                                                 // the staged inputs are no longer read
    float* red = reinterpret_cast<float*>(smem);                    // [4][64][16]
    float* zs = red + 4 * 64 * 16;                                   // [2][ZS_ROWS][128]
    if (kh == 1) {
        f32x4* rp = reinterpret_cast<f32x4*>(red + (cg * 64 + lane) * 16);
        rp[0] = ag[0];
        rp[1] = ag[1];
        rp[2] = au[0];
        rp[3] = au[1];
    }
    __syncthreads();
    if (kh == 0) {
        const f32x4* rp = reinterpret_cast<const f32x4*>(red + (cg * 64 + lane) * 16);
        const int col = cg * 32 + acc_col(lane), rb = 4 * (lane >> 4);
        const f32x4 g0 = rp[0], g1 = rp[1], u0 = rp[2], u1 = rp[3];
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (rb + r < rn) {
                zs[(rb + r) * 128 + col] = ag[0][r] + g0[r];
                zs[(rb + r) * 128 + col + 8] = ag[1][r] + g1[r];
                zs[(ZS_ROWS + rb + r) * 128 + col] = au[0][r] + u0[r];
                zs[(ZS_ROWS + rb + r) * 128 + col + 8] = au[1][r] + u1[r];
            }
    }
    __syncthreads();

    const size_t P = a.P;
    unsigned long long* cnt = a.cnt_gu + (size_t)s * (N >> 7) + cb;
    const bool part = kc1 - kc0 < KC;
    if (part) {
        // four columns per thread: one device-coherent 16-byte store / load each, through a buffer resource over the
        // (slot, matrix) block's first row (uniform), offsets (r N + c) * 4
        for (int mat = 0; mat < 2; ++mat)
            for (int i = tid; i < rn * 32; i += GU_WAVES * 64) {
                const int r = i >> 5, c = (i & 31) * 4;
                st_coh16(coh_rsrc(a.zg + ((size_t)(slot * 2 + mat) * P + row0) * N + cb * 128), 4 * (r * N + c),
                         __builtin_bit_cast(u32x4, *reinterpret_cast<const f32x4*>(zs + (mat * ZS_ROWS + r) * 128 + c)));
            }
        if (!arrive_fragment(cnt, (unsigned)(kc1 - kc0), slot, (unsigned)KC, &slot_mask, &last_flag)) return;
        const unsigned mask = slot_mask;
        for (int mat = 0; mat < 2; ++mat)
            for (int i = tid; i < rn * 32; i += GU_WAVES * 64) {
                const int r = i >> 5, c = (i & 31) * 4;
                f32x4 v = {0.f, 0.f, 0.f, 0.f};
                for (unsigned m = mask; m; m &= m - 1)              // the slots in order (the chunks in K order)
                    v += __builtin_bit_cast(
                        f32x4, ld_coh16(coh_rsrc(a.zg + ((size_t)(__builtin_ctz(m) * 2 + mat) * P + row0) * N + cb * 128),
                                        4 * (r * N + c)));
                *reinterpret_cast<f32x4*>(zs + (mat * ZS_ROWS + r) * 128 + c) = v;
            }
        __syncthreads();
    }

    // epilogue: output Hadamard, SwiGLU, down-input rotation; wave w takes rows 4w .. 4w + 3 (one per 16-lane row),
    // lane columns 8 (lane % 16) .. + 7 of the block; rows past rn repeat the last row and are not stored
    if (wv * 4 < rn) {
        // the lane's coordinates are re-derived here so nothing of the epilogue stays live across the main loop
        const int ln = opaque_lane(), eg4 = ln >> 4, el16 = ln & 15;
        const int rr = wv * 4 + eg4, r = min(rr, rn - 1);
        const int colb = cb * 128 + 8 * el16;
        if (DEPTH != 4) load_scales();
        auto half = [](const u32x4& v, int i) { return u16_as_h(v[i >> 1] >> (16 * (i & 1))); };
        const float L = a.limit;
        float g[8], u[8], bv[8];
        *reinterpret_cast<float4*>(g) = *reinterpret_cast<const float4*>(zs + r * 128 + 8 * el16);
        *reinterpret_cast<float4*>(g + 4) = *reinterpret_cast<const float4*>(zs + r * 128 + 8 * el16 + 4);
        *reinterpret_cast<float4*>(u) = *reinterpret_cast<const float4*>(zs + (ZS_ROWS + r) * 128 + 8 * el16);
        *reinterpret_cast<float4*>(u + 4) = *reinterpret_cast<const float4*>(zs + (ZS_ROWS + r) * 128 + 8 * el16 + 4);
        fwht128_x16s(g, ln);
        fwht128_x16s(u, ln);
        const float hr = HAD_R * fwht_sign(ln);                      // r and the sign fwht128_x16s leaves
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float gv = g[i] * hr * (float)half(svg, i);
            float uv = u[i] * hr * (float)half(svu, i);
            float sv = gv * sigmoid_dexp(gv);
            if (L != 0.0f) {
                sv = fminf(sv, L);
                uv = fminf(fmaxf(uv, -L), L);
            }
            const _Float16 a16 = (_Float16)(sv * uv);
            bv[i] = (float)(_Float16)(a16 * half(sud, i));
        }
        fwht128_x16s(bv, ln);
        if (rr < rn) {
            u32x4 o;
#pragma unroll
            for (int m = 0; m < 4; ++m)
                o[m] = h_as_u16((_Float16)(bv[2 * m] * hr)) | (h_as_u16((_Float16)(bv[2 * m + 1] * hr)) << 16);
            *reinterpret_cast<u32x4*>(a.xd + (size_t)(row0 + rr) * N + colb) = o;
        }
    }
    if (part && tid == 0) *cnt = 0ull;
}

template <int DEPTH, bool SHARED>
__global__ __launch_bounds__(GU_WAVES * 64) __attribute__((amdgpu_waves_per_eu(4))) void dec_gateup_kernel(
    DecodeArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    // grid (N/128, K splits, segments): split ks is chunk ks (kch_gu = K / splits), its partials in slot ks
    gateup_tile<DEPTH, SHARED>(a, blockIdx.x, blockIdx.z, blockIdx.y, blockIdx.y + 1, blockIdx.y, smem);
}

// grid (K/512, N splits, segments), 512 threads: workgroup = 512 output columns of one segment over one N range;
// wave w = columns 64w..64w+63 (column tiles 4w..4w+3: the first pair as "g", the second as "u" of the two-matrix
// step, sharing the staged input) over the whole range.
constexpr int DN_COLS = 512;
// The down tile (column block cb, N split ks, segment s) of a 512-thread workgroup; smem: the dynamic LDS.
template <int DEPTH>
__device__ __forceinline__ void down_tile(const DecodeArgs& a, int cb, int s, int kc0, int kc1, int slot,
                                          unsigned char* smem) {
    __shared__ int last_flag;
    __shared__ unsigned slot_mask;
    if (s >= a.nseg[0]) return;
    const int e = a.seg_expert[s], row0 = a.seg_row0[s], rn = a.seg_rows[s];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int K = a.K, N = a.N, KT = K >> 4;
    const int NR = (kc1 - kc0) * a.kch_dn, nbase = kc0 * a.kch_dn, RSH = NR + XPAD;
    const int NC = N / a.kch_dn;
    uint32_t* xw = reinterpret_cast<uint32_t*>(smem);              // [rn][RSD] inputs duplicated per n: (x, x)
    const int RSD = NR + 4;

    // prologue: the segment's down inputs (already rotated) for this N range, 8 halves per load; the first batch is
    // loaded unconditionally (chunk index clamped) before the weight prefetch (loads return in issue order)
    const int cpr = NR >> 3, nchunk = rn * cpr;                      // 16-byte chunks per row, in all
    constexpr int PB = 2;                                            // chunks per thread per batch
    u32x4 xv[PB];
    auto chunk_src = [&](int i) {
        i = min(i, nchunk - 1);
        const int r = i / cpr, k = 8 * (i - r * cpr);
        return *reinterpret_cast<const u32x4*>(a.xd + (size_t)(row0 + r) * N + nbase + k);
    };
    auto chunk_store = [&](int i, const u32x4& v) {
        // halves k..k+7 (k = 16 g + 8 h) go duplicated to staged dwords 4 m + 2 h, 4 m + 2 h + 1 of group g
        const int r = i / cpr, k = 8 * (i - r * cpr);
        uint32_t* d = xw + (size_t)r * RSD + (k & ~15) + 2 * ((k >> 3) & 1);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const uint32_t lo = v[m] & 0xFFFFu, hi = v[m] >> 16;
            *reinterpret_cast<uint2*>(d + 4 * m) = make_uint2(lo | (lo << 16), hi | (hi << 16));
        }
    };
#pragma unroll
    for (int c = 0; c < PB; ++c) xv[c] = chunk_src(tid + c * DN_WAVES * 64);
    __builtin_amdgcn_sched_barrier(0);

    const int t = lane >> 3, q = lane & 7;
    const int ct = cb * (DN_COLS / 16) + wv * 4 + (t & 1);
    const u32x4* D = reinterpret_cast<const u32x4*>(a.wt.d_tr[e]);
    const size_t sstr = (size_t)KT * 8 * 4;
    const size_t idx0 = ((size_t)((nbase >> 4) + (t >> 1)) * KT + ct) * 8 + q;
    const int steps = NR >> 6;                                       // a multiple of DEPTH
    // K % 256 == 0: in the last workgroup the upper waves may have no columns (wave-uniform; they only stage)
    // (their prefetch re-reads column tiles 0..3 so that every wave issues the same loads)
    const bool live = cb * DN_COLS + wv * 64 < K;
    const size_t pf0 = live ? idx0 : ((size_t)((nbase >> 4) + (t >> 1)) * KT + (t & 1)) * 8 + q;
    u32x4 gb[DEPTH], ub[DEPTH];                                      // column tiles ct and ct + 2
#pragma unroll
    for (int j = 0; j < DEPTH; ++j) {
        gb[j] = ld_stream(D + pf0 + j * sstr);
        ub[j] = ld_stream(D + pf0 + 16 + j * sstr);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int c = 0; c < PB; ++c)
        if (tid + c * DN_WAVES * 64 < nchunk) chunk_store(tid + c * DN_WAVES * 64, xv[c]);
    for (int i0 = tid + PB * DN_WAVES * 64; i0 < nchunk; i0 += PB * DN_WAVES * 64) {
#pragma unroll
        for (int c = 0; c < PB; ++c) xv[c] = chunk_src(i0 + c * DN_WAVES * 64);
#pragma unroll
        for (int c = 0; c < PB; ++c)
            if (i0 + c * DN_WAVES * 64 < nchunk) chunk_store(i0 + c * DN_WAVES * 64, xv[c]);
    }
    __syncthreads();

    const int arow = min(lane & 15, rn - 1);
    const uint32_t* xr = xw + (size_t)arow * RSD + (t >> 1) * 16;
    f32x4 ag[2], au[2];
    ag[0] = ag[1] = au[0] = au[1] = f32x4{0.f, 0.f, 0.f, 0.f};
    u32x4 xa[4], xn[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) xa[i] = reinterpret_cast<const u32x4*>(xr)[i];
    uint32_t pg = prev_word(gb[0][3], lane), pu = prev_word(ub[0][3], lane);
    for (int q = 0, st = 0; live && q < 4; ++q) {
      prio_for_quarter(q);
      for (const int st1 = quarter_end<DEPTH>(q, steps); st < st1; st += DEPTH) {
#pragma unroll
        for (int j = 0; j < DEPTH; ++j) {
            const size_t nx = idx0 + (size_t)min(st + DEPTH + j, steps - 1) * sstr;
            const int sn = min(st + j + 1, steps - 1);
            const int jn = (j + 1) % DEPTH;
            const uint32_t pgn = prev_word(gb[jn][3], lane), pun = prev_word(ub[jn][3], lane);
#pragma unroll
            for (int i = 0; i < 4; ++i) xn[i] = reinterpret_cast<const u32x4*>(xr + sn * 64)[i];
            step_mfma2_dup(gb[j], pg, ub[j], pu, xa, ag, au);
            gb[j] = ld_stream(D + nx);
            ub[j] = ld_stream(D + nx + 16);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < 4; ++i) xa[i] = xn[i];
            pg = pgn;
            pu = pun;
        }
      }
    }
    __builtin_amdgcn_s_setprio(0);
    // this wave's first epilogue task (below): its column scales and row factors are loaded here, so their latency
    // overlaps the staging of the sums and any split-N reduction
    const int ncol = min(DN_COLS, K - cb * DN_COLS);                // 256 or 512
    const int NBLK = ncol / 128, ntk = rn * NBLK;
    u32x4 svd0 = {};
    uint16_t w16_0 = 0;
    int pe_0 = -1;
    if (4 * wv < ntk) {
        const int l = opaque_lane(), tc = min(4 * wv + (l >> 4), ntk - 1), r = tc / NBLK;
        svd0 = ld_g128(reinterpret_cast<const _Float16*>(a.wt.d_svh[e]) + cb * DN_COLS + (tc - r * NBLK) * 128 +
                       8 * (l & 15));
        w16_0 = a.w16[row0 + r];
        pe_0 = a.pe[row0 + r];
    }
    __syncthreads();                                                 // the staged inputs are no longer read
    float* zs = reinterpret_cast<float*>(smem);                     // [ZS_ROWS][DN_COLS]
    {
        const int col = wv * 64 + acc_col(lane), rb = 4 * (lane >> 4);
#pragma unroll
        for (int r = 0; r < 4; ++r)
            if (live && rb + r < rn) {
                zs[(rb + r) * DN_COLS + col] = ag[0][r];
                zs[(rb + r) * DN_COLS + col + 8] = ag[1][r];
                zs[(rb + r) * DN_COLS + col + 32] = au[0][r];
                zs[(rb + r) * DN_COLS + col + 40] = au[1][r];
            }
    }
    __syncthreads();

    const size_t P = a.P;
    unsigned long long* cnt = a.cnt_dn + (size_t)s * ((K + DN_COLS - 1) / DN_COLS) + cb;
    const bool part = kc1 - kc0 < NC;
    if (part) {
        // four columns per thread (ncol is a multiple of 4), as in the gate/up kernel
        for (int i = tid; i < rn * (DN_COLS / 4); i += DN_WAVES * 64) {
            const int r = i / (DN_COLS / 4), c = (i % (DN_COLS / 4)) * 4;
            if (c < ncol)
                st_coh16(coh_rsrc(a.zd + ((size_t)slot * P + row0) * K + cb * DN_COLS), 4 * (r * K + c),
                         __builtin_bit_cast(u32x4, *reinterpret_cast<const f32x4*>(zs + r * DN_COLS + c)));
        }
        if (!arrive_fragment(cnt, (unsigned)(kc1 - kc0), slot, (unsigned)NC, &slot_mask, &last_flag)) return;
        const unsigned mask = slot_mask;
        for (int i = tid; i < rn * (DN_COLS / 4); i += DN_WAVES * 64) {
            const int r = i / (DN_COLS / 4), c = (i % (DN_COLS / 4)) * 4;
            if (c >= ncol) continue;
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            for (unsigned m = mask; m; m &= m - 1)                  // the slots in order (the chunks in N order)
                v += __builtin_bit_cast(
                    f32x4, ld_coh16(coh_rsrc(a.zd + ((size_t)__builtin_ctz(m) * P + row0) * K + cb * DN_COLS),
                                    4 * (r * K + c)));
            *reinterpret_cast<f32x4*>(zs + r * DN_COLS + c) = v;
        }
        __syncthreads();
    }

    // epilogue: (row, 128-column block) tasks, four per wave at a time (one per 16-lane row, 8 columns per lane);
    // output Hadamard, scale, then atomics or the per-pair contribution
    const int ln = opaque_lane(), g4 = ln >> 4, l16 = ln & 15;
    for (int t0 = 4 * wv; t0 < ntk; t0 += 4 * DN_WAVES) {
        const int task = t0 + g4, tc = min(task, ntk - 1);
        const int r = tc / NBLK, hb = tc - r * NBLK;
        const size_t row = row0 + r;
        const int col = cb * DN_COLS + hb * 128 + 8 * l16;
        const bool first = t0 == 4 * wv;                             // (uniform) its loads were issued above
        const u32x4 svd = first ? svd0 : ld_g128(reinterpret_cast<const _Float16*>(a.wt.d_svh[e]) + col);
        const uint16_t w16v = first ? w16_0 : a.w16[row];
        const int pev = first ? pe_0 : a.pe[row];
        float v[8];
        *reinterpret_cast<float4*>(v) = *reinterpret_cast<const float4*>(zs + r * DN_COLS + hb * 128 + 8 * l16);
        *reinterpret_cast<float4*>(v + 4) = *reinterpret_cast<const float4*>(zs + r * DN_COLS + hb * 128 + 8 * l16 + 4);
        fwht128_x16s(v, ln);
        const float rs = HAD_R * fwht_sign(ln) * (float)u16_as_h(w16v);   // with the sign fwht128_x16s leaves
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = v[i] * rs * (float)u16_as_h(svd[i >> 1] >> (16 * (i & 1)));
        if (task < ntk && pev >= 0) {                                // pe < 0: a row whose token id was out of range
            if (a.accumulate) {
                float* o = reinterpret_cast<float*>(a.out) + (size_t)a.tok[row] * a.out_stride + col;
#pragma unroll
                for (int i = 0; i < 8; ++i) atomicAdd(o + i, v[i]);
            } else {
                float4* o = reinterpret_cast<float4*>(a.contrib + row * K + col);
                o[0] = make_float4(v[0], v[1], v[2], v[3]);
                o[1] = make_float4(v[4], v[5], v[6], v[7]);
            }
        }
    }
    if (part && tid == 0) *cnt = 0ull;
}

template <int DEPTH>
__global__ __launch_bounds__(DN_WAVES * 64) __attribute__((amdgpu_waves_per_eu(4))) void dec_down_kernel(
    DecodeArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    // grid (K/512, N splits, segments): split ks is chunk ks (kch_dn = N / splits), its partials in slot ks
    down_tile<DEPTH>(a, blockIdx.x, blockIdx.z, blockIdx.y, blockIdx.y + 1, blockIdx.y, smem);
}

// grid (T, K/256), 128 threads x 2 columns: out[t] = sum over slots k (in order) of the valid pairs' contributions
__global__ __launch_bounds__(128) void combine_kernel(DecodeArgs a) {
    const int t = blockIdx.x;
    const int col = blockIdx.y * 256 + 2 * threadIdx.x;
    float s0 = 0.f, s1 = 0.f;
    // eight slots at a time, each level of loads issued together: positions, then validity and contributions (a
    // slot's contribution row is loaded whether or not it is valid; only valid ones are added, in slot order)
    for (int k0 = 0; k0 < a.topk; k0 += 8) {
        int pos[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) pos[k] = a.inv[t * a.topk + min(k0 + k, a.topk - 1)];
        int pv[8];
        float2 c[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            pv[k] = a.pe[pos[k]];
            c[k] = *reinterpret_cast<const float2*>(a.contrib + (size_t)pos[k] * a.K + col);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k)
            if (k0 + k < a.topk && pv[k] >= 0) {
                s0 += c[k].x;
                s1 += c[k].y;
            }
    }
    const size_t o = (size_t)t * a.out_stride + col;
    if (a.out_accumulate) {                                          // out += the routed sum (one rounding)
        if (a.odt == DT_F32) {
            s0 += reinterpret_cast<const float*>(a.out)[o];
            s1 += reinterpret_cast<const float*>(a.out)[o + 1];
        } else if (a.odt == DT_BF16) {
            s0 += bf16_to_f32(reinterpret_cast<const uint16_t*>(a.out)[o]);
            s1 += bf16_to_f32(reinterpret_cast<const uint16_t*>(a.out)[o + 1]);
        } else {
            s0 += (float)reinterpret_cast<const _Float16*>(a.out)[o];
            s1 += (float)reinterpret_cast<const _Float16*>(a.out)[o + 1];
        }
    }
    if (a.odt == DT_F32) {
        *reinterpret_cast<float2*>(reinterpret_cast<float*>(a.out) + o) = make_float2(s0, s1);
    } else if (a.odt == DT_BF16) {
        const uint32_t v = pack_bf16x2(s0, s1);
        *reinterpret_cast<uint32_t*>(reinterpret_cast<uint16_t*>(a.out) + o) = v;
    } else {
        *reinterpret_cast<h2*>(reinterpret_cast<uint16_t*>(a.out) + o) = h2{(_Float16)s0, (_Float16)s1};
    }
}

// ------------------------------------------------------------------------------------------------ sigmoid

// The epilogues' logistic sigmoid on n values (grid-stride): variant 0 = sigmoid_dexp (decode epilogue), 1 =
// sigmoid_fast (grouped prefill epilogues).
__global__ __launch_bounds__(256) void sigmoid_kernel(const float* __restrict__ g, int64_t n, int variant,
                                                      float* __restrict__ out) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        out[i] = variant ? sigmoid_fast(g[i]) : sigmoid_dexp(g[i]);
}

// ------------------------------------------------------------------------------------------------ launchers

int launch_sigmoid(const float* g, int64_t n, int variant, float* out, hipStream_t st) {
    const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>((n + 255) / 256, 8192));
    hipLaunchKernelGGL(sigmoid_kernel, dim3((unsigned)blocks), dim3(256), 0, st, g, n, variant, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_dequant(const uint16_t* trellis, int kt, int nt, uint16_t* wq, hipStream_t st) {
    hipLaunchKernelGGL(dequant_kernel, dim3(nt / 8, kt), dim3(64), 0, st, reinterpret_cast<const u32x4*>(trellis), nt,
                       wq);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_rot_in(const void* x, int xdt, int64_t x_stride, const int* tok, const int* pe, const int64_t* suh_tab,
                  int P, int K, uint16_t* out, hipStream_t st) {
    hipLaunchKernelGGL(rot_in_kernel, dim3(P, K / 128), dim3(64), 0, st, x, xdt, x_stride, tok, pe, suh_tab, K, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

size_t decode_lds_gateup(int rmax, int kr, int shared_suh) {
    size_t staged = (size_t)(shared_suh ? 1 : 2) * rmax * (kr + XPAD) * 2;
    if (shared_suh) staged = std::max(staged, (size_t)std::min(rmax, DUP_ROWS) * (kr + 4) * 4);
    const size_t reduce = (size_t)(4 * 64 * 16 + 2 * ZS_ROWS * 128) * 4;
    return std::max(staged, reduce);
}
size_t decode_lds_down(int rmax, int kr) {
    return std::max((size_t)rmax * (kr + 4) * 4, (size_t)ZS_ROWS * DN_COLS * 4);
}


template <typename F>
static int allow_lds(F* f) {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(f), hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)DECODE_LDS_MAX) == hipSuccess ? 0 : -1;
}

static int decode_setup() {
    static bool done = false;
    if (done) return 0;
    if (allow_lds(dec_gateup_kernel<4, true>) || allow_lds(dec_gateup_kernel<2, true>) ||
        allow_lds(dec_gateup_kernel<4, false>) || allow_lds(dec_gateup_kernel<2, false>) ||
        allow_lds(dec_down_kernel<4>) || allow_lds(dec_down_kernel<2>))
        return -1;
    done = true;
    return 0;
}

int launch_decode(const DecodeArgs& a0, int rmax, hipStream_t st, int kernels) {
    if (rmax < 1 || rmax > ZS_ROWS) return 1;
    if (decode_setup()) return -1;
    DecodeArgs a = a0;
    a.rmax = rmax;
    // load depth: four steps (of 64 k) when each wave's range holds a multiple of four, else two
    if (kernels & 1) {
        const dim3 grid(a.N / 128, a.sk_gu, a.S_cap);
        const size_t lds = decode_lds_gateup(rmax, a.kch_gu, a.shared_suh);
        const bool d4 = ((a.kch_gu / 2) >> 6) % 4 == 0;
        if (a.shared_suh) {
            if (d4) hipLaunchKernelGGL((dec_gateup_kernel<4, true>), grid, dim3(GU_WAVES * 64), lds, st, a);
            else hipLaunchKernelGGL((dec_gateup_kernel<2, true>), grid, dim3(GU_WAVES * 64), lds, st, a);
        } else {
            if (d4) hipLaunchKernelGGL((dec_gateup_kernel<4, false>), grid, dim3(GU_WAVES * 64), lds, st, a);
            else hipLaunchKernelGGL((dec_gateup_kernel<2, false>), grid, dim3(GU_WAVES * 64), lds, st, a);
        }
    }
    if (kernels & 2) {
        const dim3 grid((a.K + DN_COLS - 1) / DN_COLS, a.sk_dn, a.S_cap);
        const size_t lds = decode_lds_down(rmax, a.kch_dn);
        if ((a.kch_dn >> 6) % 4 == 0)
            hipLaunchKernelGGL(dec_down_kernel<4>, grid, dim3(DN_WAVES * 64), lds, st, a);
        else
            hipLaunchKernelGGL(dec_down_kernel<2>, grid, dim3(DN_WAVES * 64), lds, st, a);
    }
    if ((kernels & 4) && !a.accumulate) hipLaunchKernelGGL(combine_kernel, dim3(a.T, a.K / 256), dim3(128), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace mi355moe
