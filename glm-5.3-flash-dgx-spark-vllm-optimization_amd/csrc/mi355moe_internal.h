// Internal launch descriptors shared by the kernel files and the C-ABI layer (host and device visible).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mi355moe {

enum DType { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

constexpr int ROUTE_SMALL_MAX_P = 1024;   // pairs the one-block permutation handles

// Permutation of P = T * topk routed pairs into expert order.
struct RouteArgs {
    const void* ids;        // [P] int32 or int64 router ids
    int ids64;
    const void* w;          // [P] router weights (wdt)
    int wdt;
    const int64_t* emap;    // optional expert map [n_global] (global id -> local id or -1)
    int64_t n_global;
    int P, topk, n, R, seg, S_cap;
    int Rmin;               // experts with count <= Rmin get no rows (pe = -1) and no segments (0: none excluded)
    // outputs (sorted position order unless noted)
    int* tok;               // [P] token of the pair at pos
    uint16_t* w16;          // [P] fp16 weight bits
    float* w32;             // optional [P] fp32 weight
    int* pe;                // [P] local expert, -1 = skipped (sentinel, more than R or at most Rmin rows)
    int* inv;               // [P] pair j -> pos
    int* seg_expert;        // [S_cap]
    int* seg_row0;          // [S_cap]
    int* seg_rows;          // [S_cap]
    int* nseg;              // [1]
    int* counts;            // optional [n + 1] pairs per local id (last = sentinel)
    // multi-block scratch
    int* loc;               // [P]
    int* blk_cnt;           // [ceil(P / 1024) * (n + 1)]
    int* cnt_out;           // [n + 1]
    // split-K arrival counters of the kernels that follow, zeroed by the first route kernel of the call
    unsigned* zero;
    int64_t zero_words;
};

// Pointer tables of one layer's experts: device arrays of n int64 device addresses.
struct Exl3Tables {
    const int64_t* g_tr;    // gate trellis int16 [K/16][N/16][64]
    const int64_t* g_suh;   // fp16 [K]
    const int64_t* g_svh;   // fp16 [N]
    const int64_t* u_tr;
    const int64_t* u_suh;
    const int64_t* u_svh;
    const int64_t* d_tr;    // down trellis int16 [N/16][K/16][64]
    const int64_t* d_suh;   // fp16 [N]
    const int64_t* d_svh;   // fp16 [K]
};

// The decode-path kernels (grouped trellis GEMV with fused epilogues).
struct DecodeArgs {
    Exl3Tables wt;
    int n, K, N, P, T;
    // activations
    const void* x;
    int xdt;                // DT_F16 or DT_BF16
    int64_t x_stride;       // elements
    // routing tables (sorted position order)
    const int* tok;
    const uint16_t* w16;
    const int* pe;
    const int* inv;         // pair j -> pos (slot-order combine); nullptr when pairs have no slots
    const int* seg_expert;
    const int* seg_row0;
    const int* seg_rows;
    const int* nseg;
    int S_cap;
    // Work decomposition: a tile is (row segment, column block); its reduction dimension (K for gate/up, N for
    // down) is cut into sk_gu / sk_dn chunks of kch_gu / kch_dn elements, one workgroup per chunk (grid (column
    // blocks, chunks, segments)). A tile computed in more than one chunk is summed by the chunk that arrives last,
    // in chunk order.
    int sk_gu, sk_dn;
    int kch_gu, kch_dn;     // chunk length (K elements for gate/up, N elements for down)
    int rmax;               // rows per segment (<= 16)
    int shared_suh;         // gate and up share one input rotation (one staged copy)
    float limit;
    // workspace
    float* zg;              // [K / kch_gu][2][P][N] partial sums, slot = the fragment's first chunk
    float* zd;              // [N / kch_dn][P][K]
    uint16_t* xd;           // [P][N] fp16 bits
    float* contrib;         // [P][K] per-pair contribution (slot-order combine)
    unsigned long long* cnt_gu;   // [S_cap][N/128]: chunks arrived (bits 0-31) | slots stored (bits 32-63); zero
    unsigned long long* cnt_dn;   // [S_cap][ceil(K/512)]                                           between calls
    // output
    void* out;
    int odt;                // output dtype
    int64_t out_stride;
    int accumulate;         // 1: out (fp32) += contributions with atomics; 0: out = slot-order sum
    int topk;
    int out_accumulate;     // with accumulate 0: out += the slot-order sum (the shared-expert fold)
};

// The prefill-path kernels (gather, fp16 MFMA grouped GEMMs over 256-row expert tiles).
struct PrefillArgs {
    Exl3Tables wt;
    int n, K, N, P, T;
    const void* x;
    int xdt;
    int64_t x_stride;
    const int* tok;
    const uint16_t* w16;
    const int* pe;
    const int* seg_expert;
    const int* seg_row0;
    const int* seg_rows;
    const int* nseg;
    int S_cap;
    float limit;
    uint16_t* h13;          // [P][K] rotated gate/up inputs
    uint16_t* h2;           // [P][N] rotated down inputs
    float* contrib;         // [P][K] per-pair raw down accumulators (sorted position order)
    const int* inv;         // [P] pair j -> sorted position
    int topk;
    void* out;
    int odt;
    int64_t out_stride;
    // the trellis-sourced e4m3 variant (e4m3 = 1; 0: the E3 fp16 numerics, these pointers unused)
    int e4m3;
    float* asc;             // [P] row scales of the gate/up inputs
    float* dsc;             // [P] row scales of the down inputs (nullptr: no scaling in the combine)
    float* vd;              // [P][N] fp32 down inputs before their quantization
    unsigned* amaxd;        // [P] row maxima of |vd| (float bits)
    const float* w32;       // [P] fp32 router weights for the combine (nullptr: the fp16 w16)
    // gathers over caller-built tables (the stage entries): work item i is row i with token tok64[i] (instead of
    // tok) for i < nrows[0] (device count; nullptr: all P), or, with pair_pos, routed pair i = (token i / topk, slot
    // i % topk) with local expert pair_local[i] (>= n or < 0: skipped) written to row pair_pos[i]
    const int64_t* tok64;
    const int* nrows;
    const int* pair_local;
    const int* pair_pos;
    // thin/fat split: rows with pe < 0 and pe_thin >= 0 were computed by the decode kernels, whose contrib rows hold
    // finished contributions (the combine adds them as they are); nullptr: no split
    const int* pe_thin;
    // every expert shares one w13 suh: h13 (and, e4m3, asc) hold one row per token, row pos reads token tok[pos]'s
    int tok_rows;
    int contrib_bf16;       // the down kernel stores its raw accumulators as bf16 (contrib viewed as bf16 [P][K])
    int out_accumulate;     // the combine adds the routed sum to out's current values (the shared-expert fold)
    int small_rows;         // > 0: segments of at most this many rows go to the small-tile GEMMs, larger ones to the
                            // 256-row GEMMs (set by launch_prefill; 0: one kind takes every segment)
    // the e4m3 extension's stage entries (caller-owned buffers in that extension's byte layout: one e4m3 code per
    // element, columns in the staging order of h13 / h2)
    uint8_t* a8out;         // e4m3 gathers: the rows' e4m3 codes [rows][K] instead of their fp16 values in h13
    uint8_t* a8dout;        // e4m3 down-input quantization: also the codes [P][N] of the down inputs
    uint16_t* a16out;       // e4m3 gate/up: also the fp16 SwiGLU output [P][N] in plain column order
    int down16;             // e4m3 gate/up writes the fp16 rotated down input h2 for an fp16 down GEMM (the
                            // extension's DOWN16 variant) instead of vd / amaxd
    int chunk, nchunks;     // nchunks > 1: the GEMMs and row kernels take only the segments
                            // [ns chunk / nchunks, ns (chunk + 1) / nchunks) of the ns = nseg[0] live ones
    const int* row_expert;  // optional: the row-table setup marks row r with row_expert[r] instead of its segment's
    // one-launch schedule (nullptr: separate gate/up and down launches): control words [PF_SCHED_WORDS(S_cap)] --
    // the next ticket of queue q at [PF_SCHED_QSTRIDE q] (q < PF_SCHED_QUEUES), the give-up word after them (set
    // when a down item gave up waiting), then from PF_SCHED_HEAD per (segment, part) the gate/up items finished -- zeroed by
    // the gather that starts the call; sched_lag: the schedule's lag in segments of a queue (0: all of them);
    // sched_force: always (otherwise launch_prefill takes the schedule for calls on the 256-row tiles only)
    int* sched;
    int sched_lag;
    int sched_force;
};
constexpr int PREFILL_TM = 256;
constexpr int PF_SCHED_QUEUES = 8;      // ticket queues (one per XCD; segment s in queue s % 8)
constexpr int PF_SCHED_QSTRIDE = 32;    // words between queue counters (one 128-byte line each)
constexpr int PF_SCHED_HEAD = PF_SCHED_QUEUES * PF_SCHED_QSTRIDE + PF_SCHED_QSTRIDE;
// control words of a call with S_cap segments: the head, then a count per (segment, part), up to four 64-row parts
__host__ __device__ constexpr int64_t PF_SCHED_WORDS(int64_t S_cap) { return PF_SCHED_HEAD + 4 * S_cap; }

// Item t of the one-launch gate/up -> down schedule over ns segments with ncg gate/up and ncd down items each
// (column blocks), lag L = min(lag, ns) (lag <= 0: ns): the gate/up items of segments 0 .. L - 1, then for
// r = 0 .. ns - L - 1 the gate/up items of segment L + r followed by the down items of segment r, then the down items
// of segments ns - L .. ns - 1 (the reference's item order, code/fork/kernels/moe_e4m3.cu:867-872, 931-959).
// Every down item of a segment comes after all of that segment's gate/up items, so a down item only waits for items
// with smaller tickets, which workgroups already running hold. kind: 0 gate/up, 1 down, -1 past the last item.
struct PfSchedItem {
    int kind, seg, block;
};
__host__ __device__ inline PfSchedItem pf_sched_item(int64_t t, int ns, int lag, int ncg, int ncd) {
    PfSchedItem r{-1, 0, 0};
    if (t < 0 || ns <= 0 || ncg <= 0 || ncd <= 0) return r;
    const int64_t L = (lag <= 0 || lag > ns) ? ns : lag;
    const int64_t round = ncg + ncd;
    const int64_t lead = L * ncg, mid = (ns - L) * round;
    if (t < lead) {
        r.kind = 0;
        r.seg = (int)(t / ncg);
        r.block = (int)(t % ncg);
    } else if (t < lead + mid) {
        const int64_t u = t - lead, q = u / round, w = u % round;
        if (w < ncg) {
            r.kind = 0;
            r.seg = (int)(L + q);
            r.block = (int)w;
        } else {
            r.kind = 1;
            r.seg = (int)q;
            r.block = (int)(w - ncg);
        }
    } else if (t < lead + mid + L * ncd) {
        const int64_t u = t - lead - mid;
        r.kind = 1;
        r.seg = (int)(ns - L + u / ncd);
        r.block = (int)(u % ncd);
    }
    return r;
}
constexpr int PF_ROWS_PER_TOKEN = 32;   // rows of one token the row-table combine handles (topk <= 32)

// kernels: bit 0 gather, bit 1 gate/up, bit 2 down (e4m3: the down-input quantization, then the down GEMM), bit 3
// slot-order combine into the output dtype; PF_NO_QUANTD with bit 2: h2 already holds the down inputs
constexpr int PF_NO_QUANTD = 16;
int launch_prefill(const PrefillArgs& a, hipStream_t st, int kernels);
// A call over caller-built row tables (rows a.P = rows_cap, segments a.seg_* / a.nseg, chunk a.chunk / a.nchunks):
// the rows the live segments cover are marked in pe (their segment's expert, or a.row_expert[r]), every other row -1;
// then optionally e4m3 code rows widened into the GEMMs' fp16 staging (a8 -> a8_dst: every row < a8_rows, or only the
// marked ones), launch_prefill's `kernels` over the marked rows, and with tokens > 0 every token's marked rows
// (row_token) summed in row order and ADDED to out (fp32 or bf16 [tokens][K], row stride a.out_stride) with the row
// weights a.w32 (fp32) or a.w16 (fp16). tok32 (optional): [P] the rows' tokens as int32 (outside [0, tokens): 0), for
// token-row A operands. cnt [tokens], list [tokens][PF_ROWS_PER_TOKEN] and pe [P] are scratch.
struct RowsPlan {
    int* pe;
    const int64_t* row_token;
    int tokens;
    int* cnt;
    int2* list;
    int* tok32;
    const uint8_t* a8;
    int a8_rows, a8_cols, a8_all;
    uint16_t* a8_dst;
    int kernels;
};
int launch_prefill_rows(const PrefillArgs& a, const RowsPlan& p, hipStream_t st);
// out[t][0 .. K) = 0 for t < a.T (a.out, a.odt F32 or BF16, a.out_stride)
int launch_zero_out(const PrefillArgs& a, hipStream_t st);
int prefill_setup();

// The block-scaled e4m3 expert path: per-token e4m3 activations, grouped GEMMs over 64-row segments (e4m3 operands
// converted to fp16, exact products, fp32 block sums on the fp16 matrix cores).
struct Fp8Args {
    int n, K, N, P, T;
    const uint8_t* w13;     // [n][2N][K] e4m3, gate rows then up rows
    const float* w13s;      // [n][2N/128][K/128]
    const uint8_t* w2;      // [n][K][N] e4m3
    const float* w2s;       // [n][K/128][N/128]
    const void* x;
    int xdt;                // DT_F32, DT_F16 or DT_BF16
    int64_t x_stride;
    const int* tok;
    const float* w32;
    const int* pe;
    const int* seg_expert;
    const int* seg_row0;
    const int* seg_rows;
    const int* nseg;
    int S_cap;
    float limit;
    uint8_t* qx;            // [T][K] e4m3 activations
    float* sx;              // [T] their scales
    uint16_t* a16;          // [P][N] fp16 SwiGLU output (sorted position order)
    uint8_t* qa;            // [P][N] e4m3 down inputs
    float* sa;              // [P]
    float* contrib;         // [P][K] per-pair weighted contribution (sorted position order)
    const int* inv;         // [P] pair j -> sorted position
    int topk;
    void* out;
    int odt;
    int64_t out_stride;
};
constexpr int FP8_TM = 64;   // rows per segment (two 32-row MFMA tiles)
// kernels: bit 0 quantize inputs, bit 1 gate/up, bit 2 down-input quantization + down, bit 3 slot-order combine
int launch_fp8(const Fp8Args& a, hipStream_t st, int kernels);
int launch_quant_rows(const void* x, int xdt, int64_t stride, int rows, int K, uint8_t* q, float* s, hipStream_t st);

int launch_router_logits(const uint16_t* x, int64_t x_stride, const uint16_t* w, int T, int K, int E, float* logits,
                         hipStream_t st);
int launch_router_topk(const float* logits, int T, int E, const float* bias, int topk, float scale, int renorm,
                       int32_t* ids, float* wts, hipStream_t st);
int launch_route(const RouteArgs& a, hipStream_t st);
// segment tables of rows grouped by expert from int64 counts [n] (n <= 4096), ceil(count / tile) segments each
int launch_seg_tables(const int64_t* counts, int n, int tile, int max_segs, int* se, int* sr0, int* sr, int* ns,
                      int* nr, hipStream_t st);
// fat-expert row tables of the grouped tier (counts > cap, back to back in expert order); sc: int scratch [2 n]
int launch_fat_tables(const int64_t* counts, int n, int cap, const int64_t* token_sorted,
                      const uint16_t* weight_sorted, int rows_cap, int tile, int max_segs, int* se, int* sr0, int* sr,
                      int* ns, int* nr, int* row_expert, int64_t* row_token, uint16_t* row_weight, int* sc,
                      hipStream_t st);
// the permutation (a.w32, a.counts required) and the e4m3 extension's plan tables from it
int launch_route_rows(const RouteArgs& a, int* local, int* pos, int64_t* row_token, float* row_weight,
                      int* row_expert, int64_t* counts64, hipStream_t st);
// top-k of T tokens' logits and the permutation of the picks in one workgroup (P <= ROUTE_SMALL_MAX_P, a.ids = ids)
int launch_topk_route(const float* logits, int T, int E, const float* bias, int topk, float scale, int renorm,
                      int32_t* ids, float* wts, const RouteArgs& a, hipStream_t st);
// router GEMV + top-k + permutation in one launch (bf16 x and router weight, K % 512 == 0)
int launch_router_route(const uint16_t* x, int64_t x_stride, const uint16_t* w, int K, float* logits, int T, int E,
                        const float* bias, int topk, float scale, int renorm, int32_t* ids, float* wts,
                        const RouteArgs& a, unsigned* arrivals, hipStream_t st);
int launch_route_counts(const int64_t* counts64, const int64_t* token_sorted, const uint16_t* weight_sorted, int B,
                        const RouteArgs& a, hipStream_t st);
// kernels: bit 0 gate/up, bit 1 down, bit 2 combine
int launch_decode(const DecodeArgs& a, int rmax, hipStream_t st, int kernels = 7);
// LDS bytes of the decode GEMV workgroups staging kr reduction elements (gate/up: K range, down: N range)
size_t decode_lds_gateup(int rmax, int kr, int shared_suh);
size_t decode_lds_down(int rmax, int kr);
constexpr size_t DECODE_LDS_MAX = 81920;   // two 512-thread workgroups per CU
int launch_dequant(const uint16_t* trellis, int kt, int nt, uint16_t* wq, hipStream_t st);
int launch_sigmoid(const float* g, int64_t n, int variant, float* out, hipStream_t st);
int launch_rot_in(const void* x, int xdt, int64_t x_stride, const int* tok, const int* pe, const int64_t* suh_tab,
                  int P, int K, uint16_t* out, hipStream_t st);

}  // namespace mi355moe
