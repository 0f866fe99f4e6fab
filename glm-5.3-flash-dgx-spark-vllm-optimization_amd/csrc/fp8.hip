// Block-scaled e4m3 routed experts on gfx950's fp8 matrix cores: vLLM's fp8 w8a8 block-quantised MoE layout
// (w13 [n][2N][K] and w2 [n][K][N] e4m3 with one fp32 scale per 128x128 block) with per-token dynamic e4m3
// activations -- the e4m3 expert variant of the routed-MoE layer.
//
// Numerics (the reference's e4m3 contract, code/fork/kernels/moe_e4m3.cu:1-25 and :152-176,
// code/fork/overlay/glm53_moe_e4m3.py:648-674, with block-scaled weights in place of the trellis decode):
//   quant    per row: s = amax(|v|) / 448 (1 if 0), q = e4m3_rn(clamp(v / s, -448, 448))   (IEEE divisions)
//   gate/up  acc = sum over 128-k blocks b of (sum_{k in b} q_x[k] * W8[n][k]) * ws[n/128][b]  (fp8 MFMA, fp32
//            accumulate); g = acc * s_x, u likewise; a16 = fp16(silu(min(g, L)) * clamp(u, -L, L)) (iff L != 0),
//            silu(v) = v / (1 + (float)exp(-(double)v))
//   down     q_a, s_a = quant(a16 row); y = (same GEMM with the down scales) * s_a; out[token] += w * y (fp32 atomics)
//
// Work decomposition: a workgroup (4 waves) owns one 64-row segment of one expert and 128 output columns; wave w
// owns 32 of them for both 32-row tiles (and, in gate/up, for gate and up, so the SwiGLU is local to the lane).
// Per 128-k block every lane loads 64 contiguous bytes of its weight row and of each of its two activation rows:
// lane half h = lane/32 holds k 64h..64h+63, and v_mfma_scale_f32_32x32x64_f8f6f4 #1 takes the first 32 of those
// bytes, #2 the last 32 (the same k assignment for both operands, so the dot products are the block's). The block
// sum is scaled by its weight scale in fp32 before it joins the accumulator. Loads run one block ahead.
#include "common.cuh"
#include "mi355moe_internal.h"

namespace mi355moe {

typedef int i32x8 __attribute__((ext_vector_type(8)));
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

__device__ __forceinline__ f32x16 mfma_fp8(const u32x4& a0, const u32x4& a1, const u32x4& b0, const u32x4& b1,
                                           const f32x16& c) {
    const i32x8 a = {(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
    const i32x8 b = {(int)b0[0], (int)b0[1], (int)b0[2], (int)b0[3], (int)b1[0], (int)b1[1], (int)b1[2], (int)b1[3]};
    // operand formats 0 / 0 = e4m3; scale exponents 127 = 2^0 (no scaling)
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

// The 128-k block sum of one 32x32 tile from 64-byte chunks (A rows, B columns), times its block scale, added to acc.
__device__ __forceinline__ void block_acc(const u32x4 (&xa)[4], const u32x4 (&wb)[4], float ws, f32x16& acc) {
    f32x16 p = {};
    p = mfma_fp8(xa[0], xa[1], wb[0], wb[1], p);
    p = mfma_fp8(xa[2], xa[3], wb[2], wb[3], p);
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] += p[i] * ws;
}

typedef __attribute__((address_space(1))) const u32x4 gu32x4_f8;
__device__ __forceinline__ void ld64_stream(const uint8_t* p, u32x4 (&v)[4]) {
    const gu32x4_f8* q = reinterpret_cast<gu32x4_f8*>(reinterpret_cast<uintptr_t>(p));
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = __builtin_nontemporal_load(q + i);
}
__device__ __forceinline__ void ld64(const uint8_t* p, u32x4 (&v)[4]) {
    const u32x4* q = reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = q[i];
}

// Accumulator layout of a 32x32 tile: lane l holds column l % 32, register r row 8 (r / 4) + 4 (l / 32) + r % 4.
__device__ __forceinline__ int tile_row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

// grid (N/128, segments), 256 threads: the 64-row segment's gate and up outputs of 128 columns, SwiGLU -> a16.
__global__ __launch_bounds__(256) void fp8_gateup_kernel(Fp8Args a) {
    const int cb = blockIdx.x, s = blockIdx.y;
    if (s >= a.nseg[0]) return;
    const int e = a.seg_expert[s], row0 = a.seg_row0[s], rn = a.seg_rows[s];
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int K = a.K, N = a.N, h = lane >> 5, c = lane & 31;
    const int col = cb * 128 + wv * 32 + c;
    const uint8_t* wg = a.w13 + ((size_t)e * 2 * N + col) * K + 64 * h;
    const uint8_t* wu = wg + (size_t)N * K;
    const uint8_t* x0 = a.qx + (size_t)a.tok[row0 + min(c, rn - 1)] * K + 64 * h;
    const uint8_t* x1 = a.qx + (size_t)a.tok[row0 + min(32 + c, rn - 1)] * K + 64 * h;
    const int nkb = K >> 7;
    const float* sg = a.w13s + ((size_t)e * (2 * N / 128) + cb) * nkb;
    const float* su = a.w13s + ((size_t)e * (2 * N / 128) + N / 128 + cb) * nkb;

    f32x16 g0 = {}, g1 = {}, u0 = {}, u1 = {};
    u32x4 Ag[4], Au[4], Ax0[4], Ax1[4], Bg[4], Bu[4], Bx0[4], Bx1[4];
    ld64_stream(wg, Ag);
    ld64_stream(wu, Au);
    ld64(x0, Ax0);
    ld64(x1, Ax1);
    for (int kb = 0; kb < nkb; kb += 2) {
        const size_t o1 = (size_t)min(kb + 1, nkb - 1) * 128, o2 = (size_t)min(kb + 2, nkb - 1) * 128;
        ld64_stream(wg + o1, Bg);
        ld64_stream(wu + o1, Bu);
        ld64(x0 + o1, Bx0);
        ld64(x1 + o1, Bx1);
        __builtin_amdgcn_sched_barrier(0);
        block_acc(Ax0, Ag, sg[kb], g0);
        block_acc(Ax1, Ag, sg[kb], g1);
        block_acc(Ax0, Au, su[kb], u0);
        block_acc(Ax1, Au, su[kb], u1);
        __builtin_amdgcn_sched_barrier(0);
        ld64_stream(wg + o2, Ag);
        ld64_stream(wu + o2, Au);
        ld64(x0 + o2, Ax0);
        ld64(x1 + o2, Ax1);
        __builtin_amdgcn_sched_barrier(0);
        if (kb + 1 < nkb) {
            block_acc(Bx0, Bg, sg[kb + 1], g0);
            block_acc(Bx1, Bg, sg[kb + 1], g1);
            block_acc(Bx0, Bu, su[kb + 1], u0);
            block_acc(Bx1, Bu, su[kb + 1], u1);
        }
        __builtin_amdgcn_sched_barrier(0);
    }

    const float L = a.limit;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = 32 * t + tile_row(r, lane);
            if (row < rn) {
                const int pos = row0 + row;
                const float sxv = a.sx[a.tok[pos]];
                float gv = (t ? g1[r] : g0[r]) * sxv, uv = (t ? u1[r] : u0[r]) * sxv;
                if (L != 0.0f) {
                    gv = fminf(gv, L);
                    uv = fminf(fmaxf(uv, -L), L);
                }
                const float act = __fdiv_rn(gv, 1.0f + (float)exp(-(double)gv)) * uv;
                a.a16[(size_t)pos * N + col] = (uint16_t)h_as_u16((_Float16)act);
            }
        }
    }
}

// grid (K/128, segments), 256 threads: the segment's down outputs of 128 columns, scattered with fp32 atomics.
__global__ __launch_bounds__(256) void fp8_down_kernel(Fp8Args a) {
    const int cb = blockIdx.x, s = blockIdx.y;
    if (s >= a.nseg[0]) return;
    const int e = a.seg_expert[s], row0 = a.seg_row0[s], rn = a.seg_rows[s];
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int K = a.K, N = a.N, h = lane >> 5, c = lane & 31;
    const int col = cb * 128 + wv * 32 + c;
    const uint8_t* wd = a.w2 + ((size_t)e * K + col) * N + 64 * h;
    const uint8_t* x0 = a.qa + (size_t)(row0 + min(c, rn - 1)) * N + 64 * h;
    const uint8_t* x1 = a.qa + (size_t)(row0 + min(32 + c, rn - 1)) * N + 64 * h;
    const int nkb = N >> 7;
    const float* sd = a.w2s + ((size_t)e * (K / 128) + cb) * nkb;

    f32x16 d0 = {}, d1 = {};
    u32x4 Aw[4], Ax0[4], Ax1[4], Bw[4], Bx0[4], Bx1[4];
    ld64_stream(wd, Aw);
    ld64(x0, Ax0);
    ld64(x1, Ax1);
    for (int kb = 0; kb < nkb; kb += 2) {
        const size_t o1 = (size_t)min(kb + 1, nkb - 1) * 128, o2 = (size_t)min(kb + 2, nkb - 1) * 128;
        ld64_stream(wd + o1, Bw);
        ld64(x0 + o1, Bx0);
        ld64(x1 + o1, Bx1);
        __builtin_amdgcn_sched_barrier(0);
        block_acc(Ax0, Aw, sd[kb], d0);
        block_acc(Ax1, Aw, sd[kb], d1);
        __builtin_amdgcn_sched_barrier(0);
        ld64_stream(wd + o2, Aw);
        ld64(x0 + o2, Ax0);
        ld64(x1 + o2, Ax1);
        __builtin_amdgcn_sched_barrier(0);
        if (kb + 1 < nkb) {
            block_acc(Bx0, Bw, sd[kb + 1], d0);
            block_acc(Bx1, Bw, sd[kb + 1], d1);
        }
        __builtin_amdgcn_sched_barrier(0);
    }

#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = 32 * t + tile_row(r, lane);
            if (row < rn) {
                const int pos = row0 + row;
                if (a.pe[pos] < 0) continue;                         // a row whose token id was out of range
                const float y = (t ? d1[r] : d0[r]) * a.sa[pos];
                atomicAdd(a.out32 + (size_t)a.tok[pos] * K + col, a.w32[pos] * y);
            }
        }
    }
}

__global__ __launch_bounds__(256) void fp8_zero_kernel(float* __restrict__ p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) p[i] = 0.f;
}

__global__ __launch_bounds__(256) void fp8_convert_kernel(const float* __restrict__ src, int T, int K, void* dst,
                                                          int odt, int64_t stride) {
    const int64_t n = (int64_t)T * K;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const int64_t t = i / K, c = i - t * K;
        const float v = src[i];
        if (odt == DT_F32) reinterpret_cast<float*>(dst)[t * stride + c] = v;
        else if (odt == DT_BF16) reinterpret_cast<uint16_t*>(dst)[t * stride + c] = f32_to_bf16(v);
        else reinterpret_cast<_Float16*>(dst)[t * stride + c] = (_Float16)v;
    }
}

// ------------------------------------------------------------------------------------------------ launchers

int launch_quant_rows(const void* x, int xdt, int64_t stride, int rows, int K, uint8_t* q, float* s, hipStream_t st) {
    if (rows > 0) hipLaunchKernelGGL(quant_rows_kernel, dim3(rows), dim3(256), 0, st, x, xdt, stride, K, q, s);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int launch_fp8(const Fp8Args& a, hipStream_t st, int kernels) {
    const int64_t tk = (int64_t)a.T * a.K;
    const unsigned gz = (unsigned)std::max<int64_t>(1, std::min<int64_t>((tk + 255) / 256, 8192));
    if (kernels & 1) {
        hipLaunchKernelGGL(fp8_zero_kernel, dim3(gz), dim3(256), 0, st, a.out32, tk);
        if (a.T > 0) hipLaunchKernelGGL(quant_rows_kernel, dim3(a.T), dim3(256), 0, st, a.x, a.xdt, a.x_stride, a.K,
                                        a.qx, a.sx);
    }
    if (kernels & 2) hipLaunchKernelGGL(fp8_gateup_kernel, dim3(a.N / 128, a.S_cap), dim3(256), 0, st, a);
    if (kernels & 4) {
        hipLaunchKernelGGL(quant_rows_kernel, dim3(a.P), dim3(256), 0, st, (const void*)a.a16, (int)DT_F16,
                           (int64_t)a.N, a.N, a.qa, a.sa);
        hipLaunchKernelGGL(fp8_down_kernel, dim3(a.K / 128, a.S_cap), dim3(256), 0, st, a);
    }
    if (kernels & 8) hipLaunchKernelGGL(fp8_convert_kernel, dim3(gz), dim3(256), 0, st, a.out32, a.T, a.K, a.out,
                                        a.odt, a.out_stride);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace mi355moe
