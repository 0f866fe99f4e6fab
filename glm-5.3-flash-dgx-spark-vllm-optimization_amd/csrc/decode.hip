// Decode-path kernels (few rows per expert): trellis dequant, input rotation, the grouped gate/up and down trellis
// GEMVs with their epilogues fused through split-K arrival counters, and the slot-order combine.
//
// Work decomposition of the grouped GEMVs (no MFMA: at a few rows per expert the work is a stream of 4-bit codes):
//   workgroup (128-column block cb, K split ks, row segment s): 4 waves split the split's k tiles; lane (t, q) of a
//   wave owns columns q and q+8 of tile cb*8 + t, loads 16 bytes of trellis per k tile and matrix, decodes 32
//   values in registers and accumulates them against the segment's rows with v_dot2_f32_f16. Waves reduce in
//   fixed order through LDS; each split writes its fp32 partial; the workgroup that arrives last for (s, cb) adds
//   the splits in split order and runs the epilogue. Every result is therefore independent of scheduling.
// Numerics (oracle/csrc/oracle.c mode 0):
//   rot_in   xg = fp16(H(fp16(x * suh_g)) * r)                       (exl3.cu:321-349)
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

// acc[r][0..1] += the decoded tile (two columns per lane) times rows r < rn of xs (16 k values at koff)
template <int RMAX>
__device__ __forceinline__ void tile_fma(const u32x4& w, int lane, const _Float16* xs, int ldx, int koff, int rn,
                                         float (&acc)[RMAX][2]) {
    const uint32_t pw0 = prev_word(w[3], lane);
    h2 d[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) decode_word(i ? w[i - 1] : pw0, w[i], d[i]);
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
        if (r < rn) {
            const h2* xp = reinterpret_cast<const h2*>(xs + (size_t)r * ldx + koff);
            h2 xv[8];
#pragma unroll
            for (int m = 0; m < 8; ++m) xv[m] = xp[m];
            float a0 = acc[r][0], a1 = acc[r][1];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                a0 = __builtin_amdgcn_fdot2(d[i][0], xv[i], a0, false);
                a0 = __builtin_amdgcn_fdot2(d[i][1], xv[4 + i], a0, false);
                a1 = __builtin_amdgcn_fdot2(d[i][2], xv[i], a1, false);
                a1 = __builtin_amdgcn_fdot2(d[i][3], xv[4 + i], a1, false);
            }
            acc[r][0] = a0;
            acc[r][1] = a1;
        }
    }
}

// Streamed weight load: a global-address-space 16-byte load marked non-temporal (read once per call).
typedef __attribute__((address_space(1))) const u32x4 gu32x4;
__device__ __forceinline__ u32x4 ld_stream(const u32x4* p) {
    return __builtin_nontemporal_load(reinterpret_cast<gu32x4*>(reinterpret_cast<uintptr_t>(p)));
}

// Cross-wave reduction of acc (fixed order w = 0..3) and store of this split's partial rows into dst (row stride ld).
template <int RMAX>
__device__ __forceinline__ void reduce_store(float (&acc)[RMAX][2], float* red, int wv, int lane, int rn, float* dst,
                                             size_t ld) {
    const int t = lane >> 3, q = lane & 7;
#pragma unroll
    for (int r = 0; r < RMAX; ++r)
        if (r < rn) {
            red[(wv * RMAX + r) * 128 + t * 16 + q] = acc[r][0];
            red[(wv * RMAX + r) * 128 + t * 16 + q + 8] = acc[r][1];
        }
    __syncthreads();
    for (int idx = threadIdx.x; idx < rn * 128; idx += DEC_WAVES * 64) {
        const int r = idx >> 7, c = idx & 127;
        float s = red[r * 128 + c];
#pragma unroll
        for (int w2 = 1; w2 < DEC_WAVES; ++w2) s += red[(w2 * RMAX + r) * 128 + c];
        st_coherent(dst + (size_t)r * ld + c, s);
    }
    __syncthreads();
}


template <int RMAX>
__global__ __launch_bounds__(DEC_WAVES * 64) void dec_gateup_kernel(DecodeArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int last_flag;
    const int cb = blockIdx.x, ks = blockIdx.y, s = blockIdx.z;
    if (s >= a.nseg[0]) return;
    const int e = a.seg_expert[s], row0 = a.seg_row0[s], rn = a.seg_rows[s];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int K = a.K, N = a.N, NT = N >> 4;
    const int KR = K / a.sk_gu, kbase = ks * KR;
    _Float16* xs = reinterpret_cast<_Float16*>(smem);              // [2][RMAX][KR]

    // prologue: the segment's rotated gate and up inputs for this K range
    const int nb = KR >> 7;
    for (int task = wv; task < rn * 2 * nb; task += DEC_WAVES) {
        const int r = task / (2 * nb), rem = task - r * 2 * nb, mat = rem / nb, b = rem - mat * nb;
        const _Float16* suh = reinterpret_cast<const _Float16*>((mat ? a.wt.u_suh : a.wt.g_suh)[e]) + kbase + b * 128;
        rot_in_block(a.x, a.xdt, (size_t)a.tok[row0 + r] * a.x_stride + kbase + b * 128, suh,
                     xs + (size_t)(mat * RMAX + r) * KR + b * 128, lane);
    }
    __syncthreads();

    // main loop: this wave's k tiles of gate and up
    const int t = lane >> 3, q = lane & 7;
    const int KTw = (KR >> 4) / DEC_WAVES;
    const int ktl0 = wv * KTw;                                       // local k tile (within KR)
    const u32x4* G = reinterpret_cast<const u32x4*>(a.wt.g_tr[e]);
    const u32x4* U = reinterpret_cast<const u32x4*>(a.wt.u_tr[e]);
    const size_t kstr = (size_t)NT * 8;
    size_t idx = ((size_t)((kbase >> 4) + ktl0) * NT + cb * 8 + t) * 8 + q;
    float ag[RMAX][2], au[RMAX][2];
#pragma unroll
    for (int r = 0; r < RMAX; ++r) ag[r][0] = ag[r][1] = au[r][0] = au[r][1] = 0.f;
    // software pipeline: the next two k tiles of both matrices are in flight while the current two are decoded
    u32x4 g0 = ld_stream(G + idx), u0 = ld_stream(U + idx);
    u32x4 g1 = ld_stream(G + idx + kstr), u1 = ld_stream(U + idx + kstr);
    for (int kk = 0; kk < KTw; kk += 2) {
        idx += 2 * kstr;
        u32x4 ng0 = g0, nu0 = u0, ng1 = g1, nu1 = u1;
        if (kk + 2 < KTw) {
            ng0 = ld_stream(G + idx);
            nu0 = ld_stream(U + idx);
            ng1 = ld_stream(G + idx + kstr);
            nu1 = ld_stream(U + idx + kstr);
        }
        const int koff = (ktl0 + kk) * 16;
        tile_fma<RMAX>(g0, lane, xs, KR, koff, rn, ag);
        tile_fma<RMAX>(u0, lane, xs + (size_t)RMAX * KR, KR, koff, rn, au);
        tile_fma<RMAX>(g1, lane, xs, KR, koff + 16, rn, ag);
        tile_fma<RMAX>(u1, lane, xs + (size_t)RMAX * KR, KR, koff + 16, rn, au);
        g0 = ng0;
        u0 = nu0;
        g1 = ng1;
        u1 = nu1;
    }
    __syncthreads();                                                 // xs is reused for the reduction

    float* red = reinterpret_cast<float*>(smem);                    // [DEC_WAVES][RMAX][128]
    const size_t P = a.P;
    reduce_store<RMAX>(ag, red, wv, lane, rn, a.zg + ((size_t)(ks * 2 + 0) * P + row0) * N + cb * 128, N);
    reduce_store<RMAX>(au, red, wv, lane, rn, a.zg + ((size_t)(ks * 2 + 1) * P + row0) * N + cb * 128, N);

    unsigned* cnt = a.cnt_gu + (size_t)s * (N >> 7) + cb;
    if (!arrive_last(cnt, (unsigned)a.sk_gu, &last_flag)) return;

    // epilogue (last split): sum the splits in order, output Hadamard, SwiGLU, down-input rotation
    const int col = cb * 128 + 2 * lane;
    const h2 svg = *reinterpret_cast<const h2*>(reinterpret_cast<const _Float16*>(a.wt.g_svh[e]) + col);
    const h2 svu = *reinterpret_cast<const h2*>(reinterpret_cast<const _Float16*>(a.wt.u_svh[e]) + col);
    const h2 sud = *reinterpret_cast<const h2*>(reinterpret_cast<const _Float16*>(a.wt.d_suh[e]) + col);
    const float L = a.limit;
    for (int r = wv; r < rn; r += DEC_WAVES) {
        const size_t row = row0 + r;
        float g[2] = {0.f, 0.f}, u[2] = {0.f, 0.f};
        for (int k = 0; k < a.sk_gu; ++k) {
            const float* zg = a.zg + ((size_t)(k * 2) * P + row) * N + col;
            const float* zu = a.zg + ((size_t)(k * 2 + 1) * P + row) * N + col;
            g[0] += ld_coherent(zg);
            g[1] += ld_coherent(zg + 1);
            u[0] += ld_coherent(zu);
            u[1] += ld_coherent(zu + 1);
        }
        fwht128_w64(g[0], g[1], lane);
        fwht128_w64(u[0], u[1], lane);
        float b[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const float gv = g[i] * HAD_R * (float)(i ? svg.y : svg.x);
            float uv = u[i] * HAD_R * (float)(i ? svu.y : svu.x);
            float sv = gv * sigmoid_dexp(gv);
            if (L != 0.0f) {
                sv = fminf(sv, L);
                uv = fminf(fmaxf(uv, -L), L);
            }
            const _Float16 a16 = (_Float16)(sv * uv);
            b[i] = (float)(_Float16)(a16 * (i ? sud.y : sud.x));
        }
        fwht128_w64(b[0], b[1], lane);
        *reinterpret_cast<h2*>(a.xd + row * N + col) = h2{(_Float16)(b[0] * HAD_R), (_Float16)(b[1] * HAD_R)};
    }
    if (tid == 0) *cnt = 0u;
}

template <int RMAX>
__global__ __launch_bounds__(DEC_WAVES * 64) void dec_down_kernel(DecodeArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int last_flag;
    const int cb = blockIdx.x, ks = blockIdx.y, s = blockIdx.z;
    if (s >= a.nseg[0]) return;
    const int e = a.seg_expert[s], row0 = a.seg_row0[s], rn = a.seg_rows[s];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int K = a.K, N = a.N, KT = K >> 4;
    const int NR = N / a.sk_dn, nbase = ks * NR;
    _Float16* xs = reinterpret_cast<_Float16*>(smem);              // [RMAX][NR]
    for (int i = tid; i < rn * (NR >> 3); i += DEC_WAVES * 64) {
        const int r = i / (NR >> 3), c8 = i - r * (NR >> 3);
        *reinterpret_cast<u32x4*>(xs + (size_t)r * NR + c8 * 8) =
            *reinterpret_cast<const u32x4*>(a.xd + (size_t)(row0 + r) * N + nbase + c8 * 8);
    }
    __syncthreads();

    const int t = lane >> 3, q = lane & 7;
    const int NTw = (NR >> 4) / DEC_WAVES;
    const int ntl0 = wv * NTw;
    const u32x4* D = reinterpret_cast<const u32x4*>(a.wt.d_tr[e]);
    const size_t nstr = (size_t)KT * 8;
    size_t idx = ((size_t)((nbase >> 4) + ntl0) * KT + cb * 8 + t) * 8 + q;
    float ad[RMAX][2];
#pragma unroll
    for (int r = 0; r < RMAX; ++r) ad[r][0] = ad[r][1] = 0.f;
    u32x4 d0 = ld_stream(D + idx), d1 = ld_stream(D + idx + nstr);
    for (int kk = 0; kk < NTw; kk += 2) {
        idx += 2 * nstr;
        u32x4 n0 = d0, n1 = d1;
        if (kk + 2 < NTw) {
            n0 = ld_stream(D + idx);
            n1 = ld_stream(D + idx + nstr);
        }
        const int koff = (ntl0 + kk) * 16;
        tile_fma<RMAX>(d0, lane, xs, NR, koff, rn, ad);
        tile_fma<RMAX>(d1, lane, xs, NR, koff + 16, rn, ad);
        d0 = n0;
        d1 = n1;
    }
    __syncthreads();
    float* red = reinterpret_cast<float*>(smem);
    const size_t P = a.P;
    reduce_store<RMAX>(ad, red, wv, lane, rn, a.zd + ((size_t)ks * P + row0) * K + cb * 128, K);

    unsigned* cnt = a.cnt_dn + (size_t)s * (K >> 7) + cb;
    if (!arrive_last(cnt, (unsigned)a.sk_dn, &last_flag)) return;

    const int col = cb * 128 + 2 * lane;
    const h2 svd = *reinterpret_cast<const h2*>(reinterpret_cast<const _Float16*>(a.wt.d_svh[e]) + col);
    for (int r = wv; r < rn; r += DEC_WAVES) {
        const size_t row = row0 + r;
        if (a.pe[row] < 0) continue;                                 // a row whose token id was out of range
        float v[2] = {0.f, 0.f};
        for (int k = 0; k < a.sk_dn; ++k) {
            const float* z = a.zd + ((size_t)k * P + row) * K + col;
            v[0] += ld_coherent(z);
            v[1] += ld_coherent(z + 1);
        }
        fwht128_w64(v[0], v[1], lane);
        const float rs = HAD_R * (float)u16_as_h(a.w16[row]);
        v[0] = v[0] * rs * (float)svd.x;
        v[1] = v[1] * rs * (float)svd.y;
        if (a.accumulate) {
            float* o = reinterpret_cast<float*>(a.out) + (size_t)a.tok[row] * a.out_stride + col;
            atomicAdd(o, v[0]);
            atomicAdd(o + 1, v[1]);
        } else {
            *reinterpret_cast<float2*>(a.contrib + row * K + col) = make_float2(v[0], v[1]);
        }
    }
    if (tid == 0) *cnt = 0u;
}

// grid (T, K/256), 128 threads x 2 columns: out[t] = sum over slots k (in order) of the valid pairs' contributions
__global__ __launch_bounds__(128) void combine_kernel(DecodeArgs a) {
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

template <int RMAX>
static void launch_decode_r(const DecodeArgs& a, hipStream_t st, int kernels) {
    const int KR = a.K / a.sk_gu, NR = a.N / a.sk_dn;
    const size_t red = (size_t)DEC_WAVES * RMAX * 128 * sizeof(float);
    const size_t shm_gu = std::max((size_t)2 * RMAX * KR * 2, red);
    const size_t shm_dn = std::max((size_t)RMAX * NR * 2, red);
    if (kernels & 1)
        hipLaunchKernelGGL(dec_gateup_kernel<RMAX>, dim3(a.N / 128, a.sk_gu, a.S_cap), dim3(DEC_WAVES * 64), shm_gu,
                           st, a);
    if (kernels & 2)
        hipLaunchKernelGGL(dec_down_kernel<RMAX>, dim3(a.K / 128, a.sk_dn, a.S_cap), dim3(DEC_WAVES * 64), shm_dn, st,
                           a);
    if ((kernels & 4) && !a.accumulate) hipLaunchKernelGGL(combine_kernel, dim3(a.T, a.K / 256), dim3(128), 0, st, a);
}

int launch_decode(const DecodeArgs& a, int rmax, hipStream_t st, int kernels) {
    switch (rmax) {
        case 1: launch_decode_r<1>(a, st, kernels); break;
        case 2: launch_decode_r<2>(a, st, kernels); break;
        case 4: launch_decode_r<4>(a, st, kernels); break;
        case 8: launch_decode_r<8>(a, st, kernels); break;
        case 16: launch_decode_r<16>(a, st, kernels); break;
        default: return 1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace mi355moe
