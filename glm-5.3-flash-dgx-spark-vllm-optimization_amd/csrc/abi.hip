// C-ABI entry points: argument checks (all before the first launch), launch planning and workspace layout.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "../../include/mi355moe.h"
#include "common.cuh"
#include "mi355moe_internal.h"

using namespace mi355moe;

namespace {

constexpr int64_t MAX_PAIRS = 65536;
constexpr int64_t MAX_EXPERTS = 4096;
constexpr int64_t MAX_TOPK = 32;
constexpr size_t ALIGN = 256;

inline size_t align_up(size_t v) { return (v + ALIGN - 1) / ALIGN * ALIGN; }

int hip_rc(hipError_t e) { return e == hipSuccess ? 0 : -(int)e; }

int rc_launch(int r) {
    if (r == 0) return 0;
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? -1 : -(int)e;
}

// Every workspace layout starts with a control block of words that keep their value between calls (zero), at the
// same offset whatever the shapes of the calls sharing the workspace: data of one call never lands on them.
// Word 0 and words 64, 128, ..., 960: the arrival counters of the one-launch decode front end (its top-level count
// and its fifteen group counts, 256 bytes apart so that they do not share a cache line).
constexpr size_t WS_CONTROL_BYTES = 4096;

// Bump allocator over the caller's workspace (or a dry run that only measures), past the control block.
struct Carve {
    char* base;
    size_t off = WS_CONTROL_BYTES;
    explicit Carve(void* b) : base(static_cast<char*>(b)) {}
    template <typename T>
    T* take(size_t count) {
        T* p = base ? reinterpret_cast<T*>(base + off) : nullptr;
        off = align_up(off + count * sizeof(T));
        return p;
    }
};

// The decode plan for P pairs.
int shared_flag(const mi355moe_exl3_layer* L) { return (L->flags & MI355MOE_LAYER_SHARED_W13_SUH) ? 1 : 0; }
// one w13 suh for every expert (and gate == up): the grouped path gathers one row per token
int tok_rows_flag(const mi355moe_exl3_layer* L) {
    return (L->flags & MI355MOE_LAYER_SHARED_W13_SUH) && (L->flags & MI355MOE_LAYER_UNIFORM_W13_SUH) ? 1 : 0;
}

// The one-launch schedule's lag in segments of one ticket queue (pf_sched_item): MI355MOE_SCHED_LAG, default 0 = all
// of a queue's gate/up items before its first down item (a down item then rarely waits; small lags make down items
// wait for gate/up items still running).
int sched_lag() {
    const char* v = getenv("MI355MOE_SCHED_LAG");
    return v ? std::max(0, atoi(v)) : 0;
}

struct DecodePlan {
    int rmax, seg, S_cap, sk_gu, sk_dn, kch_gu, kch_dn;
};

int pow2ceil(int64_t v) {
    int p = 1;
    while (p < v && p < (1 << 30)) p <<= 1;
    return p;
}

DecodePlan plan_decode(int64_t P, int64_t rows_bound, int64_t n, int64_t K, int64_t N, int shared_suh) {
    DecodePlan d;
    d.rmax = (int)std::min<int64_t>(16, pow2ceil(std::max<int64_t>(1, rows_bound)));
    d.seg = d.rmax;
    d.S_cap = (int)(std::min(P, n) + (P + d.seg - 1) / d.seg);
    const int64_t s_est = std::max<int64_t>(1, std::min(P, n));
    // K splits: the fewest that keep the staged input rows within DECODE_LDS_MAX and still give ~target 512-thread
    // workgroups (one split needs no cross-workgroup reduction); each half of a split spans a multiple of 128
    const int64_t target = 400;
    int64_t sk = 0;
    for (int64_t c : {1, 2, 4, 8, 16}) {
        if (K % c || (K / c) % 256 || decode_lds_gateup(d.rmax, (int)(K / c), shared_suh) > DECODE_LDS_MAX) continue;
        sk = c;
        if (s_est * (N / 128) * c >= target) break;
    }
    d.sk_gu = (int)std::max<int64_t>(1, sk);
    int64_t nr = N;
    for (int64_t c : {1, 2, 4, 8}) {
        if (N % c || (N / c) % 128 || decode_lds_down(d.rmax, (int)(N / c)) > DECODE_LDS_MAX) continue;
        nr = N / c;
        if (s_est * ((K + 511) / 512) * c >= target) break;   // 512-column down workgroups
    }
    d.sk_dn = (int)(N / nr);
    d.kch_gu = (int)(K / d.sk_gu);
    d.kch_dn = (int)nr;
    return d;
}

struct DecodeWs {
    RouteArgs ra;
    DecodeArgs da;
    size_t bytes;
};

// Layout of the workspace for P pairs (route tables first, then the GEMV scratch).
void carve_decode(void* ws, int64_t P, int64_t n, int64_t K, int64_t N, const DecodePlan& p, bool with_contrib,
                  DecodeWs& w) {
    Carve c(ws);
    RouteArgs& r = w.ra;
    DecodeArgs& d = w.da;
    memset(&r, 0, sizeof(r));
    memset(&d, 0, sizeof(d));
    r.tok = c.take<int>(P);
    r.w16 = c.take<uint16_t>(P);
    r.pe = c.take<int>(P);
    r.inv = c.take<int>(P);
    r.seg_expert = c.take<int>(p.S_cap);
    r.seg_row0 = c.take<int>(p.S_cap);
    r.seg_rows = c.take<int>(p.S_cap);
    r.nseg = c.take<int>(1);
    r.counts = c.take<int>(n + 1);
    r.loc = c.take<int>(P);
    r.blk_cnt = c.take<int>(((P + 1023) / 1024) * (n + 1));
    r.cnt_out = c.take<int>(n + 1);
    d.cnt_gu = c.take<unsigned long long>((size_t)p.S_cap * (N / 128));
    d.cnt_dn = c.take<unsigned long long>((size_t)p.S_cap * ((K + 511) / 512));
    r.zero = reinterpret_cast<unsigned*>(d.cnt_gu);                  // both counter arrays, zeroed per call
    r.zero_words = (int64_t)((c.off - ((char*)d.cnt_gu - c.base)) / sizeof(unsigned));
    // partial-sum slots: one per chunk of a fragmented tile (none when every tile is one fragment)
    const int64_t zs_gu = K / p.kch_gu, zs_dn = N / p.kch_dn;
    d.zg = c.take<float>(zs_gu > 1 ? (size_t)zs_gu * 2 * P * N : 1);
    d.zd = c.take<float>(zs_dn > 1 ? (size_t)zs_dn * P * K : 1);
    d.xd = c.take<uint16_t>((size_t)P * N);
    d.contrib = with_contrib ? c.take<float>((size_t)P * K) : nullptr;
    w.bytes = c.off;
}

bool layer_ok(const mi355moe_exl3_layer* L) {
    return L && L->gate_trellis && L->gate_suh && L->gate_svh && L->up_trellis && L->up_suh && L->up_svh &&
           L->down_trellis && L->down_suh && L->down_svh;
}

int layer_shape_ok(const mi355moe_exl3_layer* L) {
    if (!layer_ok(L)) return MI355MOE_EINVAL;
    if (L->n < 1 || L->n > MAX_EXPERTS) return MI355MOE_ELIMIT;
    if (L->hidden < 256 || L->hidden % 256 || L->intermediate < 128 || L->intermediate % 128)
        return MI355MOE_ESHAPE;
    return 0;
}

Exl3Tables tables(const mi355moe_exl3_layer* L) {
    Exl3Tables t;
    t.g_tr = L->gate_trellis;
    t.g_suh = L->gate_suh;
    t.g_svh = L->gate_svh;
    t.u_tr = L->up_trellis;
    t.u_suh = L->up_suh;
    t.u_svh = L->up_svh;
    t.d_tr = L->down_trellis;
    t.d_suh = L->down_suh;
    t.d_svh = L->down_svh;
    return t;
}

int dt_act(int dt) { return dt == MI355MOE_F16 ? DT_F16 : dt == MI355MOE_BF16 ? DT_BF16 : -1; }

int fp8_layer_ok(const mi355moe_fp8_layer* L) {
    if (!L || !L->w13 || !L->w13_scale || !L->w2 || !L->w2_scale) return MI355MOE_EINVAL;
    if (L->n < 1 || L->n > MAX_EXPERTS) return MI355MOE_ELIMIT;
    if (L->hidden < 256 || L->hidden % 256 || L->intermediate < 128 || L->intermediate % 128)
        return MI355MOE_ESHAPE;
    if (L->hidden > 16384 || L->intermediate > 16384) return MI355MOE_ELIMIT;
    return 0;
}

struct Fp8Ws {
    RouteArgs ra;
    Fp8Args fa;
    size_t bytes;
};

// Layout of the e4m3 path's workspace: route tables (64-row segments), quantised activations, SwiGLU output and
// its quantisation, the per-pair fp32 contributions.
void carve_fp8(void* ws, int64_t P, int64_t T, int64_t n, int64_t K, int64_t N, Fp8Ws& w, int& S_cap) {
    Carve c(ws);
    RouteArgs& r = w.ra;
    Fp8Args& f = w.fa;
    memset(&r, 0, sizeof(r));
    memset(&f, 0, sizeof(f));
    S_cap = (int)(std::min(P, n) + (P + FP8_TM - 1) / FP8_TM);
    r.tok = c.take<int>(P);
    r.w16 = c.take<uint16_t>(P);
    r.w32 = c.take<float>(P);
    r.pe = c.take<int>(P);
    r.inv = c.take<int>(P);
    r.seg_expert = c.take<int>(S_cap);
    r.seg_row0 = c.take<int>(S_cap);
    r.seg_rows = c.take<int>(S_cap);
    r.nseg = c.take<int>(1);
    r.counts = c.take<int>(n + 1);
    r.loc = c.take<int>(P);
    r.blk_cnt = c.take<int>(((P + 1023) / 1024) * (n + 1));
    r.cnt_out = c.take<int>(n + 1);
    f.qx = c.take<uint8_t>((size_t)T * K);
    f.sx = c.take<float>(T);
    f.a16 = c.take<uint16_t>((size_t)P * N);
    f.qa = c.take<uint8_t>((size_t)P * N);
    f.sa = c.take<float>(P);
    f.contrib = c.take<float>((size_t)P * K);
    w.bytes = c.off;
}
int dt_w(int dt) {
    return dt == MI355MOE_F32 ? DT_F32 : dt == MI355MOE_F16 ? DT_F16 : dt == MI355MOE_BF16 ? DT_BF16 : -1;
}

}  // namespace

extern "C" {

int mi355moe_abi_version(void) { return MI355MOE_ABI_VERSION; }

const char* mi355moe_strerror(int code) {
    switch (code) {
        case MI355MOE_OK: return "ok";
        case MI355MOE_EINVAL: return "invalid argument (null pointer or bad flag)";
        case MI355MOE_ESHAPE: return "unsupported shape";
        case MI355MOE_ELIMIT: return "beyond a documented limit";
        case MI355MOE_EWORKSPACE: return "workspace too small";
        case MI355MOE_EDTYPE: return "unsupported dtype";
        case MI355MOE_EUNSUPPORTED: return "unsupported format variant";
        case MI355MOE_ESCRATCH:
            return "the call needs more device scratch than the allocation-free entry point's fixed array holds";
        default: return code < 0 ? "HIP launch error" : "unknown error";
    }
}

int mi355moe_exl3_dequant(const void* trellis, int64_t k_tiles, int64_t n_tiles, void* wq, hipStream_t stream) {
    if (!trellis || !wq) return MI355MOE_EINVAL;
    if (k_tiles < 1 || n_tiles < 8 || n_tiles % 8 || k_tiles > 65535 || n_tiles > (1 << 20)) return MI355MOE_ESHAPE;
    return rc_launch(launch_dequant(static_cast<const uint16_t*>(trellis), (int)k_tiles, (int)n_tiles,
                                    static_cast<uint16_t*>(wq), stream));
}

int mi355moe_sigmoid(const float* g, int64_t n, int variant, float* out, hipStream_t stream) {
    if (!g || !out || (variant != 0 && variant != 1)) return MI355MOE_EINVAL;
    if (n < 0) return MI355MOE_ESHAPE;
    if (n == 0) return 0;
    return rc_launch(launch_sigmoid(g, n, variant, out, stream));
}

int mi355moe_router_logits(const void* x, int64_t T, int64_t K, int64_t x_stride, const void* w, int64_t E,
                           float* logits, hipStream_t stream) {
    if (!x || !w || !logits) return MI355MOE_EINVAL;
    if (T < 0 || E < 1 || K < 512 || K % 512 || K > 8192 || x_stride < K || x_stride % 8) return MI355MOE_ESHAPE;
    if (T == 0) return 0;
    return rc_launch(launch_router_logits(static_cast<const uint16_t*>(x), x_stride, static_cast<const uint16_t*>(w),
                                          (int)T, (int)K, (int)E, logits, stream));
}

int mi355moe_router_topk(const float* logits, int64_t T, int64_t E, const float* bias, int64_t topk,
                         float routed_scale, int renormalize, int32_t* topk_ids, float* topk_weights,
                         hipStream_t stream) {
    if (!logits || !topk_ids || !topk_weights) return MI355MOE_EINVAL;
    if (E < 1 || E > 1024 || topk < 1 || topk > MAX_TOPK || topk > E || T < 0) return MI355MOE_ELIMIT;
    if (T == 0) return 0;
    return rc_launch(launch_router_topk(logits, (int)T, (int)E, bias, (int)topk, routed_scale, renormalize ? 1 : 0,
                                        topk_ids, topk_weights, stream));
}

int64_t mi355moe_route_workspace_bytes(int64_t P, int64_t n) {
    if (P < 0 || n < 0) return -1;
    return (int64_t)(WS_CONTROL_BYTES + align_up((size_t)P * 4) + align_up(((size_t)(P + 1023) / 1024) * (n + 1) * 4) +
                     align_up((size_t)(n + 1) * 4));
}

int mi355moe_route(const void* ids, int ids_dtype, const void* weights, int weights_dtype, int64_t T, int64_t topk,
                   const int64_t* expert_map, int64_t n_global, int64_t n, int64_t R, int64_t seg_rows,
                   int32_t* tok, uint16_t* w16, int32_t* pe, int32_t* inv, int32_t* seg_expert, int32_t* seg_row0,
                   int32_t* seg_rows_out, int64_t s_cap, int32_t* nseg, int32_t* counts, void* workspace,
                   size_t workspace_bytes, hipStream_t stream) {
    if (!ids || !weights || !tok || !w16 || !pe || !inv || !seg_expert || !seg_row0 || !seg_rows_out || !nseg)
        return MI355MOE_EINVAL;
    if (ids_dtype != MI355MOE_I32 && ids_dtype != MI355MOE_I64) return MI355MOE_EDTYPE;
    if (dt_w(weights_dtype) < 0) return MI355MOE_EDTYPE;
    if (T < 0 || topk < 1 || topk > MAX_TOPK || n < 1 || n > MAX_EXPERTS || R < 1 || seg_rows < 1 ||
        seg_rows > 4096)
        return MI355MOE_ELIMIT;
    if (expert_map && n_global < 0) return MI355MOE_EINVAL;
    const int64_t P = T * topk;
    if (P > MAX_PAIRS) return MI355MOE_ELIMIT;
    if (P == 0) return 0;
    if (s_cap < std::min(P, n) + (P + seg_rows - 1) / seg_rows) return MI355MOE_ESHAPE;
    const int64_t need = mi355moe_route_workspace_bytes(P, n);
    if (P > ROUTE_SMALL_MAX_P && (!workspace || (int64_t)workspace_bytes < need)) return MI355MOE_EWORKSPACE;
    RouteArgs a;
    memset(&a, 0, sizeof(a));
    a.ids = ids;
    a.ids64 = ids_dtype == MI355MOE_I64;
    a.w = weights;
    a.wdt = dt_w(weights_dtype);
    a.emap = expert_map;
    a.n_global = expert_map ? n_global : 0;
    a.P = (int)P;
    a.topk = (int)topk;
    a.n = (int)n;
    a.R = (int)std::min<int64_t>(R, 1 << 30);
    a.seg = (int)seg_rows;
    a.S_cap = (int)s_cap;
    a.tok = tok;
    a.w16 = w16;
    a.pe = pe;
    a.inv = inv;
    a.seg_expert = seg_expert;
    a.seg_row0 = seg_row0;
    a.seg_rows = seg_rows_out;
    a.nseg = nseg;
    a.counts = counts;
    if (workspace) {
        Carve c(workspace);
        a.loc = c.take<int>(P);
        a.blk_cnt = c.take<int>(((P + 1023) / 1024) * (n + 1));
        a.cnt_out = c.take<int>(n + 1);
    }
    return rc_launch(launch_route(a, stream));
}

int64_t mi355moe_route_rows_workspace_bytes(int64_t P, int64_t n) {
    if (P < 0 || n < 0) return -1;
    Carve c(nullptr);
    const int64_t S = std::min(P, n) + (P + PREFILL_TM - 1) / PREFILL_TM;
    c.take<int>(P);                  // tok
    c.take<uint16_t>(P);             // w16
    c.take<float>(P);                // w32
    c.take<int>(P);                  // pe
    c.take<int>(P);                  // inv
    c.take<int>(3 * S + 1);          // segments (unused) and their count
    c.take<int>(n + 1);              // counts
    c.take<int>(P);                  // multi-block scratch
    c.take<int>(((P + 1023) / 1024) * (n + 1));
    c.take<int>(n + 1);
    return (int64_t)c.off;
}

int mi355moe_route_rows(const void* ids, int ids_dtype, const void* weights, int weights_dtype, int64_t T,
                        int64_t topk, const int64_t* expert_map, int64_t n_global, int64_t n, int32_t* local,
                        int32_t* pos, int64_t* row_token, float* row_weight, int32_t* row_expert, int64_t* counts,
                        void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (!ids || !weights || !local || !pos || !row_token || !row_weight || !row_expert || !counts || !workspace)
        return MI355MOE_EINVAL;
    if (ids_dtype != MI355MOE_I32 && ids_dtype != MI355MOE_I64) return MI355MOE_EDTYPE;
    if (dt_w(weights_dtype) < 0) return MI355MOE_EDTYPE;
    if (T < 0 || topk < 1 || topk > MAX_TOPK || n < 1 || n > MAX_EXPERTS) return MI355MOE_ELIMIT;
    if (expert_map && n_global < 0) return MI355MOE_EINVAL;
    const int64_t P = T * topk;
    if (P > MAX_PAIRS) return MI355MOE_ELIMIT;
    if ((int64_t)workspace_bytes < mi355moe_route_rows_workspace_bytes(P, n)) return MI355MOE_EWORKSPACE;
    if (P == 0) return 0;
    const int64_t S = std::min(P, n) + (P + PREFILL_TM - 1) / PREFILL_TM;
    RouteArgs a;
    memset(&a, 0, sizeof(a));
    Carve c(workspace);
    a.tok = c.take<int>(P);
    a.w16 = c.take<uint16_t>(P);
    a.w32 = c.take<float>(P);
    a.pe = c.take<int>(P);
    a.inv = c.take<int>(P);
    a.seg_expert = c.take<int>(3 * S + 1);
    a.seg_row0 = a.seg_expert + S;
    a.seg_rows = a.seg_row0 + S;
    a.nseg = a.seg_rows + S;
    a.counts = c.take<int>(n + 1);
    a.loc = c.take<int>(P);
    a.blk_cnt = c.take<int>(((P + 1023) / 1024) * (n + 1));
    a.cnt_out = c.take<int>(n + 1);
    a.ids = ids;
    a.ids64 = ids_dtype == MI355MOE_I64;
    a.w = weights;
    a.wdt = dt_w(weights_dtype);
    a.emap = expert_map;
    a.n_global = expert_map ? n_global : 0;
    a.P = (int)P;
    a.topk = (int)topk;
    a.n = (int)n;
    a.R = 1 << 30;
    a.seg = PREFILL_TM;
    a.S_cap = (int)S;
    return rc_launch(launch_route_rows(a, local, pos, row_token, row_weight, row_expert, counts, stream));
}

int mi355moe_e3_fat_tables(const int64_t* counts, int64_t n, int64_t cap, const int64_t* token_sorted,
                           const void* weight_sorted, int64_t rows_cap, int64_t tile, int32_t* seg_expert,
                           int32_t* seg_row0, int32_t* seg_rows, int64_t max_segs, int32_t* num_segs,
                           int32_t* num_rows, int32_t* row_expert, int64_t* row_token, void* row_weight,
                           int32_t* scratch, hipStream_t stream) {
    if (!counts || !token_sorted || !weight_sorted || !seg_expert || !seg_row0 || !seg_rows || !num_segs ||
        !num_rows || !row_expert || !row_token || !row_weight || !scratch)
        return MI355MOE_EINVAL;
    if (n < 1 || n > MAX_EXPERTS || rows_cap < 0 || rows_cap > MAX_PAIRS || cap < 0) return MI355MOE_ELIMIT;
    if (tile < 16 || tile > PREFILL_TM) return MI355MOE_ESHAPE;
    if (max_segs < (rows_cap + tile - 1) / tile + n) return MI355MOE_ESHAPE;
    return rc_launch(launch_fat_tables(counts, (int)n, (int)std::min<int64_t>(cap, 1 << 30), token_sorted,
                                       static_cast<const uint16_t*>(weight_sorted), (int)rows_cap, (int)tile,
                                       (int)std::min<int64_t>(max_segs, 1 << 30), seg_expert, seg_row0, seg_rows,
                                       num_segs, num_rows, row_expert, row_token,
                                       static_cast<uint16_t*>(row_weight), scratch, stream));
}

int mi355moe_rot_in(const void* x, int x_dtype, int64_t x_stride, int64_t K, const int32_t* tok, const int32_t* pe,
                    int64_t P, const int64_t* suh_table, void* out, hipStream_t stream) {
    if (!x || !tok || !pe || !suh_table || !out) return MI355MOE_EINVAL;
    if (dt_act(x_dtype) < 0) return MI355MOE_EDTYPE;
    if (K < 128 || K % 128 || x_stride < K || x_stride % 2 || P < 0 || P > (1 << 24)) return MI355MOE_ESHAPE;
    if (P == 0) return 0;
    return rc_launch(launch_rot_in(x, dt_act(x_dtype), x_stride, tok, pe, suh_table, (int)P, (int)K,
                                   static_cast<uint16_t*>(out), stream));
}

// ---- routed experts from router ids: decode path or grouped prefill path

namespace {

struct PrefillWs {
    RouteArgs ra;
    PrefillArgs pa;
    int* sched;             // the one-launch schedule's control words [PF_SCHED_WORDS(S_cap)]
    size_t bytes;
};

void carve_prefill(void* ws, int64_t P, int64_t T, int64_t n, int64_t K, int64_t N, PrefillWs& w, int& S_cap,
                   bool e4m3 = false) {
    Carve c(ws);
    RouteArgs& r = w.ra;
    PrefillArgs& d = w.pa;
    memset(&r, 0, sizeof(r));
    memset(&d, 0, sizeof(d));
    S_cap = (int)(std::min(P, n) + (P + PREFILL_TM - 1) / PREFILL_TM);
    r.tok = c.take<int>(P);
    r.w16 = c.take<uint16_t>(P);
    r.pe = c.take<int>(P);
    r.inv = c.take<int>(P);
    r.seg_expert = c.take<int>(S_cap);
    r.seg_row0 = c.take<int>(S_cap);
    r.seg_rows = c.take<int>(S_cap);
    r.nseg = c.take<int>(1);
    r.counts = c.take<int>(n + 1);
    r.loc = c.take<int>(P);
    r.blk_cnt = c.take<int>(((P + 1023) / 1024) * (n + 1));
    r.cnt_out = c.take<int>(n + 1);
    d.h13 = c.take<uint16_t>((size_t)P * K);
    d.h2 = c.take<uint16_t>((size_t)P * N);
    d.contrib = c.take<float>((size_t)P * K);
    w.sched = c.take<int>((size_t)PF_SCHED_WORDS(S_cap));
    if (e4m3) {
        r.w32 = c.take<float>(P);
        d.w32 = r.w32;
        d.asc = c.take<float>(P);
        d.dsc = c.take<float>(P);
        d.amaxd = c.take<unsigned>(P);
        d.vd = c.take<float>((size_t)P * N);
    }
    w.bytes = c.off;
}

int choose_path(const mi355moe_exl3_layer* L, int64_t P, int path) {
    if (path == MI355MOE_PATH_AUTO)
        return (P >= MI355MOE_PREFILL_MIN_PAIRS && (L->flags & MI355MOE_LAYER_SHARED_W13_SUH)) ? MI355MOE_PATH_PREFILL
                                                                                                 : MI355MOE_PATH_DECODE;
    return path;
}

}  // namespace

int64_t mi355moe_moe_workspace_bytes_path(const mi355moe_exl3_layer* layer, int64_t T, int64_t topk, int path) {
    if (layer_shape_ok(layer) || T < 0 || topk < 1 || topk > MAX_TOPK) return -1;
    if (path < MI355MOE_PATH_AUTO || path > MI355MOE_PATH_PREFILL) return -1;
    const int64_t P = std::max<int64_t>(1, T * topk);
    if (choose_path(layer, P, path) == MI355MOE_PATH_PREFILL) {
        PrefillWs w;
        int sc;
        carve_prefill(nullptr, P, std::max<int64_t>(1, T), layer->n, layer->hidden, layer->intermediate, w, sc);
        return (int64_t)w.bytes;
    }
    const DecodePlan p = plan_decode(P, std::max<int64_t>(1, T), layer->n, layer->hidden, layer->intermediate,
                                     shared_flag(layer));
    DecodeWs w;
    carve_decode(nullptr, P, layer->n, layer->hidden, layer->intermediate, p, true, w);
    return (int64_t)w.bytes;
}

int mi355moe_sched_item(int64_t ticket, int64_t segments, int64_t lag, int64_t gateup_items, int64_t down_items,
                        int* kind, int* segment, int* block) {
    if (!kind || !segment || !block) return MI355MOE_EINVAL;
    if (segments < 0 || segments > (1 << 24) || gateup_items < 1 || gateup_items > 1024 || down_items < 1 ||
        down_items > 1024 || lag < 0)
        return MI355MOE_EINVAL;
    const PfSchedItem r = pf_sched_item(ticket, (int)segments, (int)std::min<int64_t>(lag, 1 << 24), (int)gateup_items,
                                        (int)down_items);
    *kind = r.kind;
    *segment = r.seg;
    *block = r.block;
    return 0;
}

int64_t mi355moe_moe_workspace_bytes(const mi355moe_exl3_layer* layer, int64_t T, int64_t topk) {
    return mi355moe_moe_workspace_bytes_path(layer, T, topk, MI355MOE_PATH_AUTO);
}

int mi355moe_moe_forward_ids(const mi355moe_exl3_layer* layer, const void* x, int x_dtype, int64_t x_stride,
                             int64_t T, const void* ids, int ids_dtype, const void* weights, int weights_dtype,
                             int64_t topk, const int64_t* expert_map, int64_t n_global, float limit, void* out,
                             int out_dtype, int64_t out_stride, void* workspace, size_t workspace_bytes,
                             hipStream_t stream) {
    return mi355moe_moe_forward_ids_ex(layer, x, x_dtype, x_stride, T, ids, ids_dtype, weights, weights_dtype, topk,
                                       expert_map, n_global, limit, out, out_dtype, out_stride, workspace,
                                       workspace_bytes, MI355MOE_PATH_AUTO, MI355MOE_STAGE_ALL, stream);
}

// The decode path's plan, workspace carve and argument blocks for T tokens x topk pairs (route tables: the caller
// sets the id and weight sources).
static int prep_decode(const mi355moe_exl3_layer* layer, const void* x, int x_dtype, int64_t x_stride, int64_t T,
                       int64_t topk, float limit, void* out, int out_dtype, int64_t out_stride, void* workspace,
                       size_t workspace_bytes, DecodePlan& p, DecodeWs& w) {
    const int64_t K = layer->hidden, N = layer->intermediate, n = layer->n, P = T * topk;
    p = plan_decode(P, T, n, K, N, shared_flag(layer));
    if (p.S_cap > 65535) return MI355MOE_ELIMIT;
    carve_decode(workspace, P, n, K, N, p, true, w);
    if (workspace_bytes < w.bytes) return MI355MOE_EWORKSPACE;
    RouteArgs& r = w.ra;
    r.P = (int)P;
    r.topk = (int)topk;
    r.n = (int)n;
    r.R = 1 << 30;
    r.seg = p.seg;
    r.S_cap = p.S_cap;
    DecodeArgs& d = w.da;
    d.wt = tables(layer);
    d.n = (int)n;
    d.K = (int)K;
    d.N = (int)N;
    d.P = (int)P;
    d.T = (int)T;
    d.x = x;
    d.xdt = dt_act(x_dtype);
    d.x_stride = x_stride;
    d.tok = r.tok;
    d.w16 = r.w16;
    d.pe = r.pe;
    d.inv = r.inv;
    d.seg_expert = r.seg_expert;
    d.seg_row0 = r.seg_row0;
    d.seg_rows = r.seg_rows;
    d.nseg = r.nseg;
    d.S_cap = p.S_cap;
    d.sk_gu = p.sk_gu;
    d.sk_dn = p.sk_dn;
    d.kch_gu = p.kch_gu;
    d.kch_dn = p.kch_dn;
    d.shared_suh = shared_flag(layer);
    d.limit = limit;
    d.out = out;
    d.odt = dt_w(out_dtype);
    d.out_stride = out_stride;
    d.accumulate = 0;
    d.topk = (int)topk;
    return 0;
}

// The grouped (prefill) tier over 256-row expert tiles for validated arguments: E3's fp16 numerics, or with e4m3 the
// trellis-sourced e4m3 variant (activations quantized per row, weights rounded to e4m3).
static int run_grouped(const mi355moe_exl3_layer* layer, const void* x, int x_dtype, int64_t x_stride, int64_t T,
                       const void* ids, int ids_dtype, const void* weights, int weights_dtype, int64_t topk,
                       const int64_t* expert_map, int64_t n_global, float limit, void* out, int out_dtype,
                       int64_t out_stride, void* workspace, size_t workspace_bytes, int stages, bool e4m3,
                       int options, hipStream_t stream) {
    const int64_t K = layer->hidden, N = layer->intermediate, n = layer->n, P = T * topk;
    RouteArgs r;
    PrefillWs w;
    int S_cap;
    carve_prefill(workspace, P, T, n, K, N, w, S_cap, e4m3);
    if (workspace_bytes < w.bytes) return MI355MOE_EWORKSPACE;
    r = w.ra;
    r.seg = PREFILL_TM;
    r.S_cap = S_cap;
    PrefillArgs& d = w.pa;
    d.wt = tables(layer);
    d.n = (int)n;
    d.K = (int)K;
    d.N = (int)N;
    d.P = (int)P;
    d.T = (int)T;
    d.x = x;
    d.xdt = dt_act(x_dtype);
    d.x_stride = x_stride;
    d.tok = r.tok;
    d.w16 = r.w16;
    d.pe = r.pe;
    d.inv = r.inv;
    d.topk = (int)topk;
    d.seg_expert = r.seg_expert;
    d.seg_row0 = r.seg_row0;
    d.seg_rows = r.seg_rows;
    d.nseg = r.nseg;
    d.S_cap = S_cap;
    d.limit = limit;
    d.out = out;
    d.odt = dt_w(out_dtype);
    d.out_stride = out_stride;
    d.e4m3 = e4m3 ? 1 : 0;
    d.tok_rows = tok_rows_flag(layer);
    d.contrib_bf16 = (options & MI355MOE_OPT_BF16_CONTRIB) ? 1 : 0;
    d.out_accumulate = (options & MI355MOE_OPT_ACCUMULATE) ? 1 : 0;
    if ((stages & MI355MOE_STAGE_GATEUP) && (stages & MI355MOE_STAGE_DOWN)) {
        d.sched = w.sched;                            // gate/up and down tiles in one launch: forced, or chosen
        d.sched_lag = sched_lag();                    // by launch_prefill where it measured faster
        d.sched_force = (options & MI355MOE_OPT_PERSISTENT) ? 1 : 0;
    }
    if (e4m3 && (options & MI355MOE_OPT_DOWN16)) {   // fp16 down operands: no down-input quantisation or its scale
        d.down16 = 1;
        d.dsc = nullptr;
    }
    if (prefill_setup()) return rc_launch(-1);
    r.ids = ids;
    r.ids64 = ids_dtype == MI355MOE_I64;
    r.w = weights;
    r.wdt = dt_w(weights_dtype);
    r.emap = expert_map;
    r.n_global = expert_map ? n_global : 0;
    r.P = (int)P;
    r.topk = (int)topk;
    r.n = (int)n;
    r.R = 1 << 30;
    if (stages & MI355MOE_STAGE_ROUTE)
        if (int rc = launch_route(r, stream)) return rc_launch(rc);
    int kernels = 0;
    if (stages & MI355MOE_STAGE_GATEUP) kernels |= 1 | 2;
    if (stages & MI355MOE_STAGE_DOWN) kernels |= 4;
    if (stages & MI355MOE_STAGE_COMBINE) kernels |= 8;
    return rc_launch(launch_prefill(d, stream, kernels));
}

int mi355moe_moe_forward_ids_ex(const mi355moe_exl3_layer* layer, const void* x, int x_dtype, int64_t x_stride,
                                int64_t T, const void* ids, int ids_dtype, const void* weights, int weights_dtype,
                                int64_t topk, const int64_t* expert_map, int64_t n_global, float limit, void* out,
                                int out_dtype, int64_t out_stride, void* workspace, size_t workspace_bytes, int path,
                                int stages, hipStream_t stream) {
    return mi355moe_moe_forward_ids_opt(layer, x, x_dtype, x_stride, T, ids, ids_dtype, weights, weights_dtype, topk,
                                        expert_map, n_global, limit, out, out_dtype, out_stride, workspace,
                                        workspace_bytes, path, stages, 0, stream);
}

int mi355moe_moe_forward_ids_opt(const mi355moe_exl3_layer* layer, const void* x, int x_dtype, int64_t x_stride,
                                 int64_t T, const void* ids, int ids_dtype, const void* weights, int weights_dtype,
                                 int64_t topk, const int64_t* expert_map, int64_t n_global, float limit, void* out,
                                 int out_dtype, int64_t out_stride, void* workspace, size_t workspace_bytes, int path,
                                 int stages, int options, hipStream_t stream) {
    if (int r = layer_shape_ok(layer)) return r;
    if (!x || !ids || !weights || !out || !workspace) return MI355MOE_EINVAL;
    if (stages <= 0 || stages > MI355MOE_STAGE_ALL) return MI355MOE_EINVAL;
    if (path < MI355MOE_PATH_AUTO || path > MI355MOE_PATH_PREFILL) return MI355MOE_EINVAL;
    if (options & ~(MI355MOE_OPT_ACCUMULATE | MI355MOE_OPT_BF16_CONTRIB | MI355MOE_OPT_E4M3 | MI355MOE_OPT_PERSISTENT |
                    MI355MOE_OPT_DOWN16))
        return MI355MOE_EINVAL;
    const bool e4m3 = (options & MI355MOE_OPT_E4M3) != 0;
    if ((options & MI355MOE_OPT_DOWN16) && !e4m3) return MI355MOE_EINVAL;
    if (e4m3 && path == MI355MOE_PATH_DECODE) return MI355MOE_EINVAL;      // e4m3 numerics run on the grouped tier
    if (e4m3 && layer && layer->hidden > 4096) return MI355MOE_EUNSUPPORTED;
    if (dt_act(x_dtype) < 0 || dt_w(weights_dtype) < 0 || dt_w(out_dtype) < 0) return MI355MOE_EDTYPE;
    if (ids_dtype != MI355MOE_I32 && ids_dtype != MI355MOE_I64) return MI355MOE_EDTYPE;
    const int64_t K = layer->hidden, N = layer->intermediate, n = layer->n;
    if (T < 0 || topk < 1 || topk > MAX_TOPK) return MI355MOE_ELIMIT;
    if (x_stride < K || x_stride % 2 || out_stride < K || out_stride % 2) return MI355MOE_ESHAPE;
    if (expert_map && n_global < 0) return MI355MOE_EINVAL;
    const int64_t P = T * topk;
    if (P > MAX_PAIRS) return MI355MOE_ELIMIT;
    if (P == 0) return 0;
    const int use = e4m3 ? MI355MOE_PATH_PREFILL : choose_path(layer, P, path);
    if (use == MI355MOE_PATH_PREFILL && !(layer->flags & MI355MOE_LAYER_SHARED_W13_SUH))
        return MI355MOE_EUNSUPPORTED;                   // the grouped tier gathers once with the gate's suh
    if (use == MI355MOE_PATH_PREFILL)
        return run_grouped(layer, x, x_dtype, x_stride, T, ids, ids_dtype, weights, weights_dtype, topk, expert_map,
                           n_global, limit, out, out_dtype, out_stride, workspace, workspace_bytes, stages, e4m3,
                           options, stream);
    DecodePlan p;
    DecodeWs w;
    if (int rc = prep_decode(layer, x, x_dtype, x_stride, T, topk, limit, out, out_dtype, out_stride, workspace,
                             workspace_bytes, p, w))
        return rc;
    RouteArgs& r = w.ra;
    r.ids = ids;
    r.ids64 = ids_dtype == MI355MOE_I64;
    r.w = weights;
    r.wdt = dt_w(weights_dtype);
    r.emap = expert_map;
    r.n_global = expert_map ? n_global : 0;
    if (stages & MI355MOE_STAGE_ROUTE)
        if (int rc = launch_route(r, stream)) return rc_launch(rc);
    w.da.out_accumulate = (options & MI355MOE_OPT_ACCUMULATE) ? 1 : 0;
    return rc_launch(launch_decode(w.da, p.rmax, stream, stages >> 1));
}

// ---------------------------------------------------------------------------------------------- thin/fat split

namespace {

// Workspace of the thin/fat split: one permutation (tok, w16, inv) shared by two row sets -- experts with at most cap
// rows (decode kernels, 16-row segments, pe_thin) and the rest (grouped kernels, 256-row segments, pe_fat) -- and one
// contribution buffer both fill at sorted positions.
struct SplitWs {
    RouteArgs thin, fat;
    DecodeArgs da;
    PrefillArgs pa;
    DecodePlan dp;
    size_t bytes;
};

void carve_split(void* ws, int64_t P, int64_t T, int64_t n, int64_t K, int64_t N, int64_t cap, int shared,
                 SplitWs& w) {
    Carve c(ws);
    memset(&w.thin, 0, sizeof(w.thin));
    memset(&w.da, 0, sizeof(w.da));
    memset(&w.pa, 0, sizeof(w.pa));
    DecodePlan& p = w.dp;
    p = plan_decode(P, std::max<int64_t>(1, cap), n, K, N, shared);
    p.S_cap = (int)std::min<int64_t>(p.S_cap, n * ((std::max<int64_t>(1, cap) + p.seg - 1) / p.seg));
    const int S_fat = (int)(std::min(P, n) + (P + PREFILL_TM - 1) / PREFILL_TM);
    RouteArgs& r = w.thin;
    r.tok = c.take<int>(P);
    r.w16 = c.take<uint16_t>(P);
    r.inv = c.take<int>(P);
    r.pe = c.take<int>(P);
    r.seg_expert = c.take<int>(p.S_cap);
    r.seg_row0 = c.take<int>(p.S_cap);
    r.seg_rows = c.take<int>(p.S_cap);
    r.nseg = c.take<int>(1);
    r.counts = c.take<int>(n + 1);
    r.loc = c.take<int>(P);
    r.blk_cnt = c.take<int>(((P + 1023) / 1024) * (n + 1));
    r.cnt_out = c.take<int>(n + 1);
    r.S_cap = p.S_cap;
    r.seg = p.seg;
    w.fat = r;
    w.fat.pe = c.take<int>(P);
    w.fat.seg_expert = c.take<int>(S_fat);
    w.fat.seg_row0 = c.take<int>(S_fat);
    w.fat.seg_rows = c.take<int>(S_fat);
    w.fat.nseg = c.take<int>(1);
    w.fat.S_cap = S_fat;
    w.fat.seg = PREFILL_TM;
    DecodeArgs& d = w.da;
    d.cnt_gu = c.take<unsigned long long>((size_t)p.S_cap * (N / 128));
    d.cnt_dn = c.take<unsigned long long>((size_t)p.S_cap * ((K + 511) / 512));
    r.zero = reinterpret_cast<unsigned*>(d.cnt_gu);
    r.zero_words = (int64_t)((c.off - ((char*)d.cnt_gu - c.base)) / sizeof(unsigned));
    const int64_t zs_gu = K / p.kch_gu, zs_dn = N / p.kch_dn;
    d.zg = c.take<float>(zs_gu > 1 ? (size_t)zs_gu * 2 * P * N : 1);
    d.zd = c.take<float>(zs_dn > 1 ? (size_t)zs_dn * P * K : 1);
    d.xd = c.take<uint16_t>((size_t)P * N);
    PrefillArgs& a = w.pa;
    a.h13 = c.take<uint16_t>((size_t)P * K);
    a.h2 = c.take<uint16_t>((size_t)P * N);
    a.contrib = c.take<float>((size_t)P * K);
    d.contrib = a.contrib;
    w.bytes = c.off;
}

}  // namespace

int64_t mi355moe_moe_split_workspace_bytes(const mi355moe_exl3_layer* layer, int64_t T, int64_t topk,
                                           int64_t thin_cap) {
    if (layer_shape_ok(layer) || T < 0 || topk < 1 || topk > MAX_TOPK || thin_cap < 0) return -1;
    SplitWs w;
    carve_split(nullptr, std::max<int64_t>(1, T * topk), std::max<int64_t>(1, T), layer->n, layer->hidden,
                layer->intermediate, thin_cap, shared_flag(layer), w);
    return (int64_t)w.bytes;
}

int mi355moe_moe_forward_ids_split(const mi355moe_exl3_layer* layer, const void* x, int x_dtype, int64_t x_stride,
                                   int64_t T, const void* ids, int ids_dtype, const void* weights, int weights_dtype,
                                   int64_t topk, const int64_t* expert_map, int64_t n_global, float limit, void* out,
                                   int out_dtype, int64_t out_stride, int64_t thin_cap, void* workspace,
                                   size_t workspace_bytes, hipStream_t stream) {
    if (int r = layer_shape_ok(layer)) return r;
    if (!x || !ids || !weights || !out || !workspace) return MI355MOE_EINVAL;
    if (dt_act(x_dtype) < 0 || dt_w(weights_dtype) < 0 || dt_w(out_dtype) < 0) return MI355MOE_EDTYPE;
    if (ids_dtype != MI355MOE_I32 && ids_dtype != MI355MOE_I64) return MI355MOE_EDTYPE;
    const int64_t K = layer->hidden, N = layer->intermediate, n = layer->n;
    if (T < 0 || topk < 1 || topk > MAX_TOPK || thin_cap < 0) return MI355MOE_ELIMIT;
    if (x_stride < K || x_stride % 2 || out_stride < K || out_stride % 2) return MI355MOE_ESHAPE;
    if (expert_map && n_global < 0) return MI355MOE_EINVAL;
    if (!(layer->flags & MI355MOE_LAYER_SHARED_W13_SUH)) return MI355MOE_EUNSUPPORTED;
    const int64_t P = T * topk;
    if (P > MAX_PAIRS) return MI355MOE_ELIMIT;
    if (P == 0) return 0;
    const int64_t cap = std::min(thin_cap, P);
    SplitWs w;
    carve_split(workspace, P, T, n, K, N, cap, shared_flag(layer), w);
    if (workspace_bytes < w.bytes) return MI355MOE_EWORKSPACE;
    if (w.dp.S_cap > 65535) return MI355MOE_ELIMIT;
    if (prefill_setup()) return rc_launch(-1);
    for (RouteArgs* r : {&w.thin, &w.fat}) {
        r->ids = ids;
        r->ids64 = ids_dtype == MI355MOE_I64;
        r->w = weights;
        r->wdt = dt_w(weights_dtype);
        r->emap = expert_map;
        r->n_global = expert_map ? n_global : 0;
        r->P = (int)P;
        r->topk = (int)topk;
        r->n = (int)n;
    }
    w.thin.R = (int)cap;                                             // thin: 0 < count <= cap
    w.thin.Rmin = 0;
    w.fat.R = 1 << 30;                                               // fat: count > cap
    w.fat.Rmin = (int)cap;
    w.fat.zero = nullptr;
    w.fat.zero_words = 0;
    // (the second permutation writes the same tok / w16 / inv as the first)
    if (cap > 0)
        if (int rc = launch_route(w.thin, stream)) return rc_launch(rc);
    if (int rc = launch_route(w.fat, stream)) return rc_launch(rc);
    if (cap > 0) {
        DecodeArgs& d = w.da;
        d.wt = tables(layer);
        d.n = (int)n;
        d.K = (int)K;
        d.N = (int)N;
        d.P = (int)P;
        d.T = (int)T;
        d.x = x;
        d.xdt = dt_act(x_dtype);
        d.x_stride = x_stride;
        d.tok = w.thin.tok;
        d.w16 = w.thin.w16;
        d.pe = w.thin.pe;
        d.inv = w.thin.inv;
        d.seg_expert = w.thin.seg_expert;
        d.seg_row0 = w.thin.seg_row0;
        d.seg_rows = w.thin.seg_rows;
        d.nseg = w.thin.nseg;
        d.S_cap = w.dp.S_cap;
        d.sk_gu = w.dp.sk_gu;
        d.sk_dn = w.dp.sk_dn;
        d.kch_gu = w.dp.kch_gu;
        d.kch_dn = w.dp.kch_dn;
        d.shared_suh = shared_flag(layer);
        d.limit = limit;
        d.accumulate = 0;
        d.topk = (int)topk;
        if (int rc = launch_decode(d, w.dp.rmax, stream, 1 | 2)) return rc_launch(rc);   // contributions, no combine
    }
    PrefillArgs& a = w.pa;
    a.wt = tables(layer);
    a.n = (int)n;
    a.K = (int)K;
    a.N = (int)N;
    a.P = (int)P;
    a.T = (int)T;
    a.x = x;
    a.xdt = dt_act(x_dtype);
    a.x_stride = x_stride;
    a.tok = w.fat.tok;
    a.tok_rows = tok_rows_flag(layer);
    a.w16 = w.fat.w16;
    a.pe = w.fat.pe;
    a.inv = w.fat.inv;
    a.topk = (int)topk;
    a.seg_expert = w.fat.seg_expert;
    a.seg_row0 = w.fat.seg_row0;
    a.seg_rows = w.fat.seg_rows;
    a.nseg = w.fat.nseg;
    a.S_cap = w.fat.S_cap;
    a.limit = limit;
    a.out = out;
    a.odt = dt_w(out_dtype);
    a.out_stride = out_stride;
    a.pe_thin = cap > 0 ? w.thin.pe : nullptr;
    return rc_launch(launch_prefill(a, stream, 1 | 2 | 4 | 8));
}

// ---------------------------------------------------------------------------------------------- e4m3 variant

int64_t mi355moe_e4m3_moe_workspace_bytes(const mi355moe_exl3_layer* layer, int64_t T, int64_t topk) {
    if (layer_shape_ok(layer) || T < 0 || topk < 1 || topk > MAX_TOPK) return -1;
    const int64_t P = std::max<int64_t>(1, T * topk);
    PrefillWs w;
    int sc;
    carve_prefill(nullptr, P, std::max<int64_t>(1, T), layer->n, layer->hidden, layer->intermediate, w, sc, true);
    return (int64_t)w.bytes;
}

int mi355moe_e4m3_moe_forward_ids(const mi355moe_exl3_layer* layer, const void* x, int x_dtype, int64_t x_stride,
                                  int64_t T, const void* ids, int ids_dtype, const void* weights, int weights_dtype,
                                  int64_t topk, const int64_t* expert_map, int64_t n_global, float limit, void* out,
                                  int out_dtype, int64_t out_stride, void* workspace, size_t workspace_bytes,
                                  int stages, hipStream_t stream) {
    if (int r = layer_shape_ok(layer)) return r;
    if (!x || !ids || !weights || !out || !workspace) return MI355MOE_EINVAL;
    if (stages <= 0 || stages > MI355MOE_STAGE_ALL) return MI355MOE_EINVAL;
    if (dt_act(x_dtype) < 0 || dt_w(weights_dtype) < 0 || dt_w(out_dtype) < 0) return MI355MOE_EDTYPE;
    if (ids_dtype != MI355MOE_I32 && ids_dtype != MI355MOE_I64) return MI355MOE_EDTYPE;
    const int64_t K = layer->hidden;
    if (T < 0 || topk < 1 || topk > MAX_TOPK) return MI355MOE_ELIMIT;
    if (x_stride < K || x_stride % 2 || out_stride < K || out_stride % 2) return MI355MOE_ESHAPE;
    if (expert_map && n_global < 0) return MI355MOE_EINVAL;
    if (!(layer->flags & MI355MOE_LAYER_SHARED_W13_SUH) || K > 4096) return MI355MOE_EUNSUPPORTED;
    const int64_t P = T * topk;
    if (P > MAX_PAIRS) return MI355MOE_ELIMIT;
    if (P == 0) return 0;
    return run_grouped(layer, x, x_dtype, x_stride, T, ids, ids_dtype, weights, weights_dtype, topk, expert_map,
                       n_global, limit, out, out_dtype, out_stride, workspace, workspace_bytes, stages, true, 0,
                       stream);
}

// ---------------------------------------------------------------------------------------------- whole layer

// the router scratch after the expert path's workspace: logits [T][E], picks [T][topk] (ids, weights)
static size_t router_scratch(void* base, int64_t T, int64_t topk, int64_t E, float** logits, int32_t** ids,
                             float** wts) {
    Carve c(base);
    c.off = 0;
    float* l = c.take<float>((size_t)std::max<int64_t>(1, T * E));
    int32_t* i = c.take<int32_t>((size_t)std::max<int64_t>(1, T * topk));
    float* wv = c.take<float>((size_t)std::max<int64_t>(1, T * topk));
    if (logits) *logits = l;
    if (ids) *ids = i;
    if (wts) *wts = wv;
    return c.off;
}

int64_t mi355moe_moe_layer_workspace_bytes(const mi355moe_exl3_layer* layer, int64_t T, int64_t topk, int64_t E) {
    const int64_t base = mi355moe_moe_workspace_bytes_path(layer, T, topk, MI355MOE_PATH_AUTO);
    if (base < 0 || E < 1 || E > 1024) return -1;
    return (int64_t)(align_up((size_t)base) + router_scratch(nullptr, T, topk, E, nullptr, nullptr, nullptr));
}

int mi355moe_moe_layer(const mi355moe_exl3_layer* layer, const void* x, int x_dtype, int64_t x_stride, int64_t T,
                       const void* router_w, const float* logits, int64_t E, const float* bias, int64_t topk,
                       float routed_scale, int renormalize, float limit, void* out, int out_dtype, int64_t out_stride,
                       int32_t* ids_out, float* weights_out, void* workspace, size_t workspace_bytes,
                       hipStream_t stream) {
    if (int r = layer_shape_ok(layer)) return r;
    if (!x || !out || !workspace || (!router_w) == (!logits)) return MI355MOE_EINVAL;
    if (dt_act(x_dtype) < 0 || dt_w(out_dtype) < 0) return MI355MOE_EDTYPE;
    if (router_w && x_dtype != MI355MOE_BF16) return MI355MOE_EDTYPE;        // the router GEMV reads bf16
    const int64_t K = layer->hidden;
    if (E < 1 || E > 1024 || topk < 1 || topk > MAX_TOPK || topk > E || T < 0) return MI355MOE_ELIMIT;
    if (router_w && (K % 512 || K > 8192 || x_stride % 8)) return MI355MOE_ESHAPE;
    if (x_stride < K || x_stride % 2 || out_stride < K || out_stride % 2) return MI355MOE_ESHAPE;
    if (T * topk > MAX_PAIRS) return MI355MOE_ELIMIT;
    if (T == 0) return 0;
    const int64_t base = mi355moe_moe_workspace_bytes_path(layer, T, topk, MI355MOE_PATH_AUTO);
    const int64_t need = mi355moe_moe_layer_workspace_bytes(layer, T, topk, E);
    if (base < 0 || need < 0 || (int64_t)workspace_bytes < need) return MI355MOE_EWORKSPACE;
    float* lg;
    int32_t* ids;
    float* wts;
    unsigned* arrivals = static_cast<unsigned*>(workspace);         // control word 0
    router_scratch(static_cast<char*>(workspace) + align_up((size_t)base), T, topk, E, &lg, &ids, &wts);
    if (ids_out) ids = ids_out;
    if (weights_out) wts = weights_out;
    // router GEMV, top-k, then the routed experts from the picks
    const int64_t P = T * topk;
    const bool small = choose_path(layer, P, MI355MOE_PATH_AUTO) == MI355MOE_PATH_DECODE && P <= ROUTE_SMALL_MAX_P;
    const float* lsrc = logits;
    if (router_w && !small) {
        if (int rc = launch_router_logits(static_cast<const uint16_t*>(x), x_stride,
                                          static_cast<const uint16_t*>(router_w), (int)T, (int)K, (int)E, lg, stream))
            return rc_launch(rc);
        lsrc = lg;
    }
    if (small) {
        // decode sizes: the router GEMV (when given the weight), the top-k and the permutation in one launch (the
        // last router workgroup ranks), then the expert GEMVs and the combine
        DecodePlan p;
        DecodeWs w;
        if (int rc = prep_decode(layer, x, x_dtype, x_stride, T, topk, limit, out, out_dtype, out_stride, workspace,
                                 (size_t)base, p, w))
            return rc;
        RouteArgs& r = w.ra;
        r.ids = ids;
        r.ids64 = 0;
        r.w = wts;
        r.wdt = dt_w(MI355MOE_F32);
        r.emap = nullptr;
        r.n_global = 0;
        const int rc = router_w ? launch_router_route(static_cast<const uint16_t*>(x), x_stride,
                                                      static_cast<const uint16_t*>(router_w), (int)K, lg, (int)T,
                                                      (int)E, bias, (int)topk, routed_scale, renormalize ? 1 : 0, ids,
                                                      wts, r, arrivals, stream)
                                : launch_topk_route(lsrc, (int)T, (int)E, bias, (int)topk, routed_scale,
                                                    renormalize ? 1 : 0, ids, wts, r, stream);
        if (rc) return rc_launch(rc);
        return rc_launch(launch_decode(w.da, p.rmax, stream, MI355MOE_STAGE_ALL >> 1));
    }
    if (int rc = launch_router_topk(lsrc, (int)T, (int)E, bias, (int)topk, routed_scale, renormalize ? 1 : 0, ids, wts,
                                    stream))
        return rc_launch(rc);
    return mi355moe_moe_forward_ids_ex(layer, x, x_dtype, x_stride, T, ids, MI355MOE_I32, wts, MI355MOE_F32, topk,
                                       nullptr, 0, limit, out, out_dtype, out_stride, workspace, (size_t)base,
                                       MI355MOE_PATH_AUTO, MI355MOE_STAGE_ALL, stream);
}

// ---------------------------------------------------------------------------------------------- stage entries over
// caller-built row tables: the grouped (E3) trio and the e4m3 extension's stages

int64_t mi355moe_e3_tile_rows(void) { return PREFILL_TM; }

int mi355moe_e3_gather(const void* x, int x_dtype, int64_t x_stride, int64_t tokens, int64_t K,
                       const int64_t* row_token, const int32_t* row_expert, int64_t rows_cap, int64_t n,
                       const int64_t* suh_table, void* h13, const int32_t* num_rows, hipStream_t stream) {
    if (!x || !row_token || !row_expert || !suh_table || !h13 || !num_rows) return MI355MOE_EINVAL;
    if (dt_act(x_dtype) < 0) return MI355MOE_EDTYPE;
    if (K < 256 || K % 256 || K > 8192 || x_stride < K || x_stride % 2 || tokens < 0) return MI355MOE_ESHAPE;
    if (rows_cap < 0 || rows_cap > MAX_PAIRS || n < 1 || n > MAX_EXPERTS) return MI355MOE_ELIMIT;
    if (rows_cap == 0 || tokens == 0) return 0;
    PrefillArgs a;
    memset(&a, 0, sizeof(a));
    a.wt.g_suh = suh_table;
    a.n = (int)n;
    a.K = (int)K;
    a.P = (int)rows_cap;
    a.T = (int)tokens;
    a.x = x;
    a.xdt = dt_act(x_dtype);
    a.x_stride = x_stride;
    a.pe = row_expert;
    a.tok64 = row_token;
    a.nrows = num_rows;
    a.h13 = static_cast<uint16_t*>(h13);
    return rc_launch(launch_prefill(a, stream, 1));
}

int mi355moe_e3_gateup(const void* h13, int64_t rows_cap, int64_t K, int64_t N, int64_t n,
                       const int64_t* gate_trellis, const int64_t* up_trellis, const int64_t* gate_svh,
                       const int64_t* up_svh, const int64_t* down_suh, void* h2, const int32_t* seg_expert,
                       const int32_t* seg_row0, const int32_t* seg_rows, int64_t seg_cap, const int32_t* num_segs,
                       float act_limit, hipStream_t stream) {
    if (!h13 || !gate_trellis || !up_trellis || !gate_svh || !up_svh || !down_suh || !h2 || !seg_expert ||
        !seg_row0 || !seg_rows || !num_segs)
        return MI355MOE_EINVAL;
    if (K < 256 || K % 256 || N < 128 || N % 128) return MI355MOE_ESHAPE;
    if (rows_cap < 0 || rows_cap > MAX_PAIRS || n < 1 || n > MAX_EXPERTS || seg_cap < 0 || seg_cap > 65535)
        return MI355MOE_ELIMIT;
    if (rows_cap == 0 || seg_cap == 0) return 0;
    PrefillArgs a;
    memset(&a, 0, sizeof(a));
    a.wt.g_tr = gate_trellis;
    a.wt.u_tr = up_trellis;
    a.wt.g_svh = gate_svh;
    a.wt.u_svh = up_svh;
    a.wt.d_suh = down_suh;
    a.n = (int)n;
    a.K = (int)K;
    a.N = (int)N;
    a.P = (int)rows_cap;
    a.seg_expert = seg_expert;
    a.seg_row0 = seg_row0;
    a.seg_rows = seg_rows;
    a.nseg = num_segs;
    a.S_cap = (int)seg_cap;
    a.limit = act_limit;
    a.h13 = const_cast<uint16_t*>(static_cast<const uint16_t*>(h13));
    a.h2 = static_cast<uint16_t*>(h2);
    return rc_launch(launch_prefill(a, stream, 2));
}

namespace {
// Workspace of the row-table stages: row experts [rows], raw down accumulators [rows][K], token row counts [tokens]
// and lists [tokens][PF_ROWS_PER_TOKEN]; with e4m3 also the fp32 down inputs [rows][N], their row maxima [rows], their
// e4m3 values [rows][N] (fp16) and row scales [rows], the rows' tokens [rows] and the widened gate/up input rows
// [max(rows, tokens)][K] (fp16).
struct RowsWs {
    int* pe;
    float* contrib;
    int* cnt;
    int2* list;
    float* vd;
    unsigned* amaxd;
    uint16_t* h2;
    float* dsc;
    int* tok32;
    uint16_t* h13;
    int* sched;             // e4m3: the one-launch schedule's control words [PF_SCHED_WORDS(rows)] (segments <= rows)
    size_t bytes;
};
RowsWs carve_rows(void* ws, int64_t rows, int64_t K, int64_t N, int64_t tokens, bool e4m3) {
    Carve c(ws);
    RowsWs w;
    memset(&w, 0, sizeof(w));
    w.pe = c.take<int>(std::max<int64_t>(1, rows));
    w.contrib = c.take<float>((size_t)std::max<int64_t>(1, rows) * K);
    w.cnt = c.take<int>(std::max<int64_t>(1, tokens));
    w.list = c.take<int2>((size_t)std::max<int64_t>(1, tokens) * PF_ROWS_PER_TOKEN);
    if (e4m3) {
        w.vd = c.take<float>((size_t)std::max<int64_t>(1, rows) * N);
        w.amaxd = c.take<unsigned>(std::max<int64_t>(1, rows));
        w.h2 = c.take<uint16_t>((size_t)std::max<int64_t>(1, rows) * N);
        w.dsc = c.take<float>(std::max<int64_t>(1, rows));
        w.tok32 = c.take<int>(std::max<int64_t>(1, rows));
        w.h13 = c.take<uint16_t>((size_t)std::max<int64_t>(1, std::max(rows, tokens)) * K);
        w.sched = c.take<int>((size_t)PF_SCHED_WORDS(std::max<int64_t>(1, rows)));
    }
    w.bytes = c.off;
    return w;
}
}  // namespace

int64_t mi355moe_e3_down_workspace_bytes(int64_t rows_cap, int64_t K, int64_t tokens) {
    if (rows_cap < 0 || K < 0 || tokens < 0) return -1;
    return (int64_t)carve_rows(nullptr, rows_cap, K, 0, tokens, false).bytes;
}

int mi355moe_e3_down(const void* h2, int64_t rows_cap, int64_t K, int64_t N, int64_t n, const int64_t* down_trellis,
                     const int64_t* down_svh, float* out, int64_t tokens, int64_t out_stride,
                     const int64_t* row_token, const void* row_weight, const int32_t* seg_expert,
                     const int32_t* seg_row0, const int32_t* seg_rows, int64_t seg_cap, const int32_t* num_segs,
                     void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (!h2 || !down_trellis || !down_svh || !out || !row_token || !row_weight || !seg_expert || !seg_row0 ||
        !seg_rows || !num_segs || !workspace)
        return MI355MOE_EINVAL;
    if (K < 256 || K % 256 || N < 128 || N % 128 || out_stride < K) return MI355MOE_ESHAPE;
    if (rows_cap < 0 || rows_cap > MAX_PAIRS || n < 1 || n > MAX_EXPERTS || seg_cap < 0 || seg_cap > 65535 ||
        tokens < 0 || tokens > (1 << 24))
        return MI355MOE_ELIMIT;
    if (rows_cap == 0 || seg_cap == 0 || tokens == 0) return 0;
    const RowsWs w = carve_rows(workspace, rows_cap, K, N, tokens, false);
    if (workspace_bytes < w.bytes) return MI355MOE_EWORKSPACE;
    PrefillArgs a;
    memset(&a, 0, sizeof(a));
    a.wt.d_tr = down_trellis;
    a.wt.d_svh = down_svh;
    a.n = (int)n;
    a.K = (int)K;
    a.N = (int)N;
    a.P = (int)rows_cap;
    a.T = (int)tokens;
    a.seg_expert = seg_expert;
    a.seg_row0 = seg_row0;
    a.seg_rows = seg_rows;
    a.nseg = num_segs;
    a.S_cap = (int)seg_cap;
    a.h2 = const_cast<uint16_t*>(static_cast<const uint16_t*>(h2));
    a.pe = w.pe;
    a.contrib = w.contrib;
    a.w16 = static_cast<const uint16_t*>(row_weight);
    a.out = out;
    a.odt = DT_F32;
    a.out_stride = out_stride;
    RowsPlan rp;
    memset(&rp, 0, sizeof(rp));
    rp.pe = w.pe;
    rp.row_token = row_token;
    rp.tokens = (int)tokens;
    rp.cnt = w.cnt;
    rp.list = w.list;
    rp.kernels = 4;
    return rc_launch(launch_prefill_rows(a, rp, stream));
}

int64_t mi355moe_e4m3_tile_rows(void) { return PREFILL_TM; }

int mi355moe_e4m3_seg_tables(const int64_t* counts, int64_t n, int64_t tile, int64_t rows_cap, int32_t* seg_expert,
                             int32_t* seg_row0, int32_t* seg_rows, int64_t max_segs, int32_t* num_segs,
                             int32_t* num_rows, hipStream_t stream) {
    if (!counts || !seg_expert || !seg_row0 || !seg_rows || !num_segs || !num_rows) return MI355MOE_EINVAL;
    if (n < 1 || n > MAX_EXPERTS || rows_cap < 0 || rows_cap > MAX_PAIRS) return MI355MOE_ELIMIT;
    if (tile < 16 || tile > PREFILL_TM) return MI355MOE_ESHAPE;         // the GEMMs take at most PREFILL_TM rows
    if (max_segs < (rows_cap + tile - 1) / tile + n) return MI355MOE_ESHAPE;
    return rc_launch(launch_seg_tables(counts, (int)n, (int)tile, (int)std::min<int64_t>(max_segs, 1 << 30), seg_expert,
                                       seg_row0, seg_rows, num_segs, num_rows, stream));
}

namespace {
bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// The e4m3 gathers (per routed pair, or one row per token): validated arguments -> launch.
int e4m3_gather(const void* x, int x_dtype, int64_t x_stride, int64_t T, int64_t K, const int32_t* local,
                const int32_t* pos, int64_t topk, int64_t n, const int64_t* gate_suh, uint8_t* a8, int64_t a8_rows,
                float* asc, void* out, int out_dtype, int64_t out_stride, hipStream_t stream) {
    if (!x || !gate_suh || !a8 || !asc || (!local) != (!pos)) return MI355MOE_EINVAL;
    if (dt_act(x_dtype) < 0) return MI355MOE_EDTYPE;
    if (out && out_dtype != MI355MOE_F32 && out_dtype != MI355MOE_BF16) return MI355MOE_EDTYPE;
    if (K < 256 || K % 256 || K > 4096 || x_stride < K || x_stride % 2 || (out && out_stride < K) || !al16(a8))
        return MI355MOE_ESHAPE;
    if (T < 0 || topk < 1 || topk > MAX_TOPK || T * topk > MAX_PAIRS || n < 1 || n > MAX_EXPERTS)
        return MI355MOE_ELIMIT;
    if (a8_rows < (local ? T * topk : T)) return MI355MOE_ESHAPE;    // pos[j] < T * topk rows / one row per token
    if (T == 0) return 0;
    PrefillArgs a;
    memset(&a, 0, sizeof(a));
    a.wt.g_suh = gate_suh;
    a.n = (int)n;
    a.K = (int)K;
    a.P = (int)(local ? T * topk : T);
    a.T = (int)T;
    a.topk = (int)topk;
    a.x = x;
    a.xdt = dt_act(x_dtype);
    a.x_stride = x_stride;
    a.pair_local = local;
    a.pair_pos = pos;
    a.tok_rows = local ? 0 : 1;
    a.a8out = a8;
    a.asc = asc;
    a.e4m3 = 1;
    if (out) {
        PrefillArgs z = a;
        z.out = out;
        z.odt = dt_w(out_dtype);
        z.out_stride = out_stride;
        if (int rc = launch_zero_out(z, stream)) return rc_launch(rc);
    }
    return rc_launch(launch_prefill(a, stream, 1));
}

// The common checks and argument block of the row-table e4m3 stages (rows_cap rows, seg_cap segment entries).
int e4m3_rows_args(int64_t rows_cap, int64_t K, int64_t N, int64_t n, int64_t seg_cap, const int32_t* seg_row0,
                   const int32_t* seg_rows, const int32_t* num_segs, int64_t chunk, int64_t nchunks, PrefillArgs& a) {
    if (!seg_row0 || !seg_rows || !num_segs) return MI355MOE_EINVAL;
    if (K < 256 || K % 256 || K > 4096 || N < 128 || N % 128 || N > 4096) return MI355MOE_ESHAPE;
    if (rows_cap < 0 || rows_cap > MAX_PAIRS || n < 1 || n > MAX_EXPERTS || seg_cap < 0 || seg_cap > 65535)
        return MI355MOE_ELIMIT;
    if (nchunks < 1 || chunk < 0 || chunk >= nchunks || nchunks > 65535) return MI355MOE_EINVAL;
    memset(&a, 0, sizeof(a));
    a.n = (int)n;
    a.K = (int)K;
    a.N = (int)N;
    a.P = (int)rows_cap;
    a.seg_row0 = seg_row0;
    a.seg_rows = seg_rows;
    a.nseg = num_segs;
    a.S_cap = (int)seg_cap;
    a.chunk = (int)chunk;
    a.nchunks = (int)nchunks;
    a.e4m3 = 1;
    return 0;
}
}  // namespace

int mi355moe_e4m3_gather2(const void* x, int x_dtype, int64_t x_stride, int64_t T, int64_t K, const int32_t* local,
                          const int32_t* pos, int64_t topk, int64_t n, const int64_t* gate_suh, uint8_t* a8,
                          int64_t a8_rows, float* asc, void* out, int out_dtype, int64_t out_stride,
                          hipStream_t stream) {
    if (!local || !pos) return MI355MOE_EINVAL;
    return e4m3_gather(x, x_dtype, x_stride, T, K, local, pos, topk, n, gate_suh, a8, a8_rows, asc, out, out_dtype,
                       out_stride, stream);
}

int mi355moe_e4m3_gather_tok(const void* x, int x_dtype, int64_t x_stride, int64_t T, int64_t K,
                             const int64_t* gate_suh, uint8_t* a8, int64_t a8_rows, float* asc, void* out,
                             int out_dtype, int64_t out_stride, hipStream_t stream) {
    return e4m3_gather(x, x_dtype, x_stride, T, K, nullptr, nullptr, 1, 1, gate_suh, a8, a8_rows, asc, out, out_dtype,
                       out_stride, stream);
}

int64_t mi355moe_e4m3_stage_workspace_bytes(int64_t rows_cap, int64_t K, int64_t N, int64_t tokens) {
    if (rows_cap < 0 || K < 0 || N < 0 || tokens < 0) return -1;
    return (int64_t)carve_rows(nullptr, rows_cap, K, N, tokens, true).bytes;
}

int mi355moe_e4m3_gateup(const uint8_t* a8, const float* asc, int64_t rows_cap, int64_t K, int64_t N, int64_t n,
                         const int64_t* gate_trellis, const int64_t* up_trellis, const int64_t* gate_svh,
                         const int64_t* up_svh, void* a16, const int32_t* seg_expert, const int32_t* seg_row0,
                         const int32_t* seg_rows, int64_t seg_cap, const int32_t* num_segs, float limit, int64_t chunk,
                         int64_t nchunks, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (!a8 || !asc || !gate_trellis || !up_trellis || !gate_svh || !up_svh || !a16 || !seg_expert || !workspace)
        return MI355MOE_EINVAL;
    PrefillArgs a;
    if (int rc = e4m3_rows_args(rows_cap, K, N, n, seg_cap, seg_row0, seg_rows, num_segs, chunk, nchunks, a)) return rc;
    if (!al16(a8) || !al16(a16)) return MI355MOE_ESHAPE;
    if (rows_cap == 0 || seg_cap == 0) return 0;
    const RowsWs w = carve_rows(workspace, rows_cap, K, N, 0, true);
    if (workspace_bytes < w.bytes) return MI355MOE_EWORKSPACE;
    a.wt.g_tr = gate_trellis;
    a.wt.u_tr = up_trellis;
    a.wt.g_svh = gate_svh;
    a.wt.u_svh = up_svh;
    a.seg_expert = seg_expert;
    a.limit = limit;
    a.h13 = w.h13;
    a.asc = const_cast<float*>(asc);
    a.a16out = static_cast<uint16_t*>(a16);
    RowsPlan rp;
    memset(&rp, 0, sizeof(rp));
    rp.pe = w.pe;
    rp.a8 = a8;
    rp.a8_rows = (int)rows_cap;
    rp.a8_cols = (int)K;
    rp.a8_dst = w.h13;
    rp.kernels = 2;
    return rc_launch(launch_prefill_rows(a, rp, stream));
}

int mi355moe_e4m3_actq(const void* a16, int64_t rows_cap, int64_t N, const int32_t* row_expert, int64_t n,
                       const int64_t* down_suh, uint8_t* a8d, float* dsc, const int32_t* seg_row0,
                       const int32_t* seg_rows, int64_t seg_cap, const int32_t* num_segs, int64_t chunk,
                       int64_t nchunks, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (!a16 || !row_expert || !down_suh || !a8d || !dsc || !workspace) return MI355MOE_EINVAL;
    PrefillArgs a;
    if (int rc = e4m3_rows_args(rows_cap, 256, N, n, seg_cap, seg_row0, seg_rows, num_segs, chunk, nchunks, a))
        return rc;
    if (!al16(a16) || !al16(a8d)) return MI355MOE_ESHAPE;
    if (rows_cap == 0 || seg_cap == 0) return 0;
    const RowsWs w = carve_rows(workspace, rows_cap, 256, N, 0, true);
    if (workspace_bytes < w.bytes) return MI355MOE_EWORKSPACE;
    // the gather's quantiser over the marked rows: row r reads a16 row r (K = N wide) with expert row_expert[r]'s
    // down suh, writes a8d row r and dsc[r]
    a.K = (int)N;
    a.x = a16;
    a.xdt = DT_F16;
    a.x_stride = N;
    a.wt.g_suh = down_suh;
    a.row_expert = row_expert;
    a.a8out = a8d;
    a.asc = dsc;
    RowsPlan rp;
    memset(&rp, 0, sizeof(rp));
    rp.pe = w.pe;
    rp.kernels = 1;
    return rc_launch(launch_prefill_rows(a, rp, stream));
}

int mi355moe_e4m3_down(const uint8_t* a8d, const float* dsc, int64_t rows_cap, int64_t K, int64_t N, int64_t n,
                       const int64_t* down_trellis, const int64_t* down_svh, float* out, int64_t tokens,
                       int64_t out_stride, const int64_t* row_token, const float* row_weight,
                       const int32_t* seg_expert, const int32_t* seg_row0, const int32_t* seg_rows, int64_t seg_cap,
                       const int32_t* num_segs, int64_t chunk, int64_t nchunks, void* workspace,
                       size_t workspace_bytes, hipStream_t stream) {
    if (!a8d || !dsc || !down_trellis || !down_svh || !out || !row_token || !row_weight || !seg_expert || !workspace)
        return MI355MOE_EINVAL;
    PrefillArgs a;
    if (int rc = e4m3_rows_args(rows_cap, K, N, n, seg_cap, seg_row0, seg_rows, num_segs, chunk, nchunks, a)) return rc;
    if (!al16(a8d) || out_stride < K) return MI355MOE_ESHAPE;
    if (tokens < 0 || tokens > (1 << 24)) return MI355MOE_ELIMIT;
    if (rows_cap == 0 || seg_cap == 0 || tokens == 0) return 0;
    const RowsWs w = carve_rows(workspace, rows_cap, K, N, tokens, true);
    if (workspace_bytes < w.bytes) return MI355MOE_EWORKSPACE;
    a.T = (int)tokens;
    a.wt.d_tr = down_trellis;
    a.wt.d_svh = down_svh;
    a.seg_expert = seg_expert;
    a.h2 = w.h2;
    a.contrib = w.contrib;
    a.asc = const_cast<float*>(dsc);                 // (the e4m3 checks want a gate/up scale; unused here)
    a.dsc = const_cast<float*>(dsc);
    a.w32 = row_weight;
    a.out = out;
    a.odt = DT_F32;
    a.out_stride = out_stride;
    RowsPlan rp;
    memset(&rp, 0, sizeof(rp));
    rp.pe = w.pe;
    rp.row_token = row_token;
    rp.tokens = (int)tokens;
    rp.cnt = w.cnt;
    rp.list = w.list;
    rp.a8 = a8d;
    rp.a8_rows = (int)rows_cap;
    rp.a8_cols = (int)N;
    rp.a8_dst = w.h2;
    rp.kernels = 4 | PF_NO_QUANTD;
    return rc_launch(launch_prefill_rows(a, rp, stream));
}

int mi355moe_e4m3_fused(const uint8_t* a8, const float* asc, int64_t a8_rows, uint8_t* a8d, float* dsc, void* a16,
                        void* out, int out_dtype, int64_t tokens, int64_t out_stride, int64_t K, int64_t N, int64_t n,
                        const int64_t* gate_trellis, const int64_t* up_trellis, const int64_t* gate_svh,
                        const int64_t* up_svh, const int64_t* down_trellis, const int64_t* down_suh,
                        const int64_t* down_svh, const int64_t* row_token, const float* row_weight, int64_t rows_cap,
                        const int32_t* seg_expert, const int32_t* seg_row0, const int32_t* seg_rows, int64_t seg_cap,
                        const int32_t* num_segs, float limit, int variant, void* workspace, size_t workspace_bytes,
                        hipStream_t stream) {
    if (!a8 || !asc || !out || !gate_trellis || !up_trellis || !gate_svh || !up_svh || !down_trellis || !down_suh ||
        !down_svh || !row_token || !row_weight || !seg_expert || !workspace || (!a8d) != (!dsc))
        return MI355MOE_EINVAL;
    if (variant & ~(MI355MOE_E4M3_DOWN16 | MI355MOE_E4M3_TOKEN_ROWS | MI355MOE_E4M3_LEAN_MAINLOOP))
        return MI355MOE_EINVAL;
    if (out_dtype != MI355MOE_F32 && out_dtype != MI355MOE_BF16) return MI355MOE_EDTYPE;
    PrefillArgs a;
    if (int rc = e4m3_rows_args(rows_cap, K, N, n, seg_cap, seg_row0, seg_rows, num_segs, 0, 1, a)) return rc;
    const bool tok_rows = (variant & MI355MOE_E4M3_TOKEN_ROWS) != 0, down16 = (variant & MI355MOE_E4M3_DOWN16) != 0;
    if (!al16(a8) || (a8d && !al16(a8d)) || (a16 && !al16(a16)) || out_stride < K) return MI355MOE_ESHAPE;
    if (tokens < 0 || tokens > (1 << 24)) return MI355MOE_ELIMIT;
    if (a8_rows < (tok_rows ? tokens : rows_cap)) return MI355MOE_ESHAPE;
    if (rows_cap == 0 || seg_cap == 0 || tokens == 0) return 0;
    const RowsWs w = carve_rows(workspace, rows_cap, K, N, tokens, true);
    if (workspace_bytes < w.bytes) return MI355MOE_EWORKSPACE;
    a.T = (int)tokens;
    a.wt.g_tr = gate_trellis;
    a.wt.u_tr = up_trellis;
    a.wt.g_svh = gate_svh;
    a.wt.u_svh = up_svh;
    a.wt.d_tr = down_trellis;
    a.wt.d_suh = down_suh;
    a.wt.d_svh = down_svh;
    a.seg_expert = seg_expert;
    a.limit = limit;
    a.h13 = w.h13;
    a.h2 = w.h2;
    a.contrib = w.contrib;
    a.asc = const_cast<float*>(asc);
    a.down16 = down16 ? 1 : 0;
    a.a16out = static_cast<uint16_t*>(a16);
    if (!down16) {                                    // e4m3 down: fp32 down inputs, their maxima and quantisation
        a.vd = w.vd;
        a.amaxd = w.amaxd;
        a.dsc = dsc ? dsc : w.dsc;
        a.a8dout = a8d;
    }
    a.w32 = row_weight;
    a.out = out;
    a.odt = dt_w(out_dtype);
    a.out_stride = out_stride;
    if (tok_rows) {                                   // row r's gate/up input is a8 row row_token[r]
        a.tok_rows = 1;
        a.tok = w.tok32;
    }
    RowsPlan rp;
    memset(&rp, 0, sizeof(rp));
    rp.pe = w.pe;
    rp.row_token = row_token;
    rp.tokens = (int)tokens;
    rp.cnt = w.cnt;
    rp.list = w.list;
    rp.tok32 = tok_rows ? w.tok32 : nullptr;
    rp.a8 = a8;
    rp.a8_rows = (int)(tok_rows ? tokens : rows_cap);
    rp.a8_cols = (int)K;
    rp.a8_all = tok_rows ? 1 : 0;
    rp.a8_dst = w.h13;
    rp.kernels = 2 | 4;
    if (seg_cap <= rows_cap) {                        // the one-launch schedule where the tile choice takes it
        a.sched = w.sched;                            // (zeroed by the row-table setup)
        a.sched_lag = sched_lag();
    }
    return rc_launch(launch_prefill_rows(a, rp, stream));
}

}  // extern "C"

// ---------------------------------------------------------------------------------------------- allocation-free layer

namespace {

// The device scratch of mi355moe_moe_layer_noalloc: one array per GPU, alive until the process ends, shared by every
// call on that GPU. Host code never uses this name as an address (in host code it is only a stand-in for the symbol):
// every kernel argument and fill goes through the per-device address hipGetSymbolAddress returns.
static __device__ __align__(256) unsigned char scratch[MI355MOE_NOALLOC_SCRATCH_BYTES];

constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex g_noalloc_mu;
void* g_noalloc_ptr[NOALLOC_MAX_DEVICES];          // per device: the address of its copy of `scratch`

// zeroes the control block (the arrival counter words calls expect at zero) of a device's scratch
__global__ void zero_control_kernel(unsigned* words, int n) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) words[i] = 0u;
}

bool g_noalloc_zeroed[NOALLOC_MAX_DEVICES];        // per device: its control block was zeroed outside a capture

// The current device's scratch address, looked up with that device current the first time the device is used. Until
// a call has zeroed the control block on a stream that was not being captured, every call zeroes it on `stream`
// ahead of its own kernels (a fill kernel, not a memset node; inside a captured graph it re-zeroes words that every
// call leaves at zero anyway). nullptr with *rc set when a HIP call fails.
void* noalloc_scratch(hipStream_t stream, int* rc) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= NOALLOC_MAX_DEVICES) {
        *rc = e != hipSuccess ? -(int)e : MI355MOE_ELIMIT;
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (!g_noalloc_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            *rc = e != hipSuccess ? -(int)e : -1;
            return nullptr;
        }
        g_noalloc_ptr[dev] = p;
    }
    if (!g_noalloc_zeroed[dev]) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(stream, &cs);
        if (e != hipSuccess) {
            *rc = -(int)e;
            return nullptr;
        }
        hipLaunchKernelGGL(zero_control_kernel, dim3(1), dim3(64), 0, stream,
                           static_cast<unsigned*>(g_noalloc_ptr[dev]), (int)(WS_CONTROL_BYTES / sizeof(unsigned)));
        e = hipGetLastError();
        if (e != hipSuccess) {
            *rc = -(int)e;
            return nullptr;
        }
        if (cs == hipStreamCaptureStatusNone) g_noalloc_zeroed[dev] = true;
    }
    return g_noalloc_ptr[dev];
}

}  // namespace

extern "C" {

int mi355moe_moe_layer_noalloc(const mi355moe_exl3_layer* layer, const void* x, int x_dtype, int64_t x_stride,
                               int64_t T, const void* router_w, const float* logits, int64_t E, const float* bias,
                               int64_t topk, float routed_scale, int renormalize, float limit, void* out,
                               int out_dtype, int64_t out_stride, int32_t* ids_out, float* weights_out,
                               hipStream_t stream) {
    if (int r = layer_shape_ok(layer)) return r;
    if (!x || !out || (!router_w) == (!logits)) return MI355MOE_EINVAL;
    if (E < 1 || E > 1024 || topk < 1 || topk > MAX_TOPK || topk > E || T < 0) return MI355MOE_ELIMIT;
    if (T * topk > MAX_PAIRS) return MI355MOE_ELIMIT;
    if (T == 0) return 0;
    const int64_t need = mi355moe_moe_layer_workspace_bytes(layer, T, topk, E);
    if (need < 0) return MI355MOE_ESHAPE;
    if (need > (int64_t)MI355MOE_NOALLOC_SCRATCH_BYTES) return MI355MOE_ESCRATCH;
    int rc = 0;
    void* ws = noalloc_scratch(stream, &rc);
    if (!ws) return rc;
    return mi355moe_moe_layer(layer, x, x_dtype, x_stride, T, router_w, logits, E, bias, topk, routed_scale,
                              renormalize, limit, out, out_dtype, out_stride, ids_out, weights_out, ws,
                              (size_t)MI355MOE_NOALLOC_SCRATCH_BYTES, stream);
}

int64_t mi355moe_exl3_moe_workspace_bytes(const mi355moe_exl3_layer* layer, int64_t P) {
    if (layer_shape_ok(layer) || P < 0) return -1;
    const int64_t Pp = std::max<int64_t>(1, P);
    size_t most = 0;                                  // the plan depends on the row cap: take the largest layout
    for (int64_t rows = 1; rows <= 16; rows *= 2) {
        const DecodePlan p = plan_decode(Pp, std::min(Pp, rows), layer->n, layer->hidden, layer->intermediate,
                                         shared_flag(layer));
        DecodeWs w;
        carve_decode(nullptr, Pp, layer->n, layer->hidden, layer->intermediate, p, false, w);
        most = std::max(most, w.bytes);
    }
    return (int64_t)most;
}

int mi355moe_exl3_moe(const mi355moe_exl3_layer* layer, const void* hidden, int64_t B, float* out,
                      const int64_t* expert_count, const int64_t* token_sorted, const void* weight_sorted, int64_t P,
                      int64_t max_rows, int act_function, int k_gate, int k_up, int k_down, int gate_mcg,
                      int gate_mul1, int up_mcg, int up_mul1, int down_mcg, int down_mul1, float act_limit,
                      void* workspace, size_t workspace_bytes, hipStream_t stream) {
    if (int r = layer_shape_ok(layer)) return r;
    if (!hidden || !out || !expert_count || !token_sorted || !weight_sorted || !workspace) return MI355MOE_EINVAL;
    if (act_function != 0) return MI355MOE_EUNSUPPORTED;
    if (k_gate != 4 || k_up != 4 || k_down != 4) return MI355MOE_EUNSUPPORTED;
    if (!gate_mcg || !up_mcg || !down_mcg || gate_mul1 || up_mul1 || down_mul1) return MI355MOE_EUNSUPPORTED;
    if (B < 1 || max_rows < 1) return MI355MOE_ESHAPE;
    if (P < 0 || P > MAX_PAIRS) return MI355MOE_ELIMIT;
    if (P == 0) return 0;
    const int64_t K = layer->hidden, N = layer->intermediate, n = layer->n;
    const DecodePlan p = plan_decode(P, std::min(P, max_rows), n, K, N, shared_flag(layer));
    if (p.S_cap > 65535) return MI355MOE_ELIMIT;
    DecodeWs w;
    carve_decode(workspace, P, n, K, N, p, false, w);
    if (workspace_bytes < w.bytes) return MI355MOE_EWORKSPACE;
    RouteArgs& r = w.ra;
    r.P = (int)P;
    r.n = (int)n;
    r.R = (int)std::min<int64_t>(max_rows, 1 << 30);
    r.seg = p.seg;
    r.S_cap = p.S_cap;
    DecodeArgs& d = w.da;
    d.wt = tables(layer);
    d.n = (int)n;
    d.K = (int)K;
    d.N = (int)N;
    d.P = (int)P;
    d.T = (int)B;
    d.x = hidden;
    d.xdt = DT_F16;
    d.x_stride = K;
    d.tok = r.tok;
    d.w16 = r.w16;
    d.pe = r.pe;
    d.inv = nullptr;
    d.seg_expert = r.seg_expert;
    d.seg_row0 = r.seg_row0;
    d.seg_rows = r.seg_rows;
    d.nseg = r.nseg;
    d.S_cap = p.S_cap;
    d.sk_gu = p.sk_gu;
    d.sk_dn = p.sk_dn;
    d.kch_gu = p.kch_gu;
    d.kch_dn = p.kch_dn;
    d.shared_suh = shared_flag(layer);
    d.limit = act_limit;
    d.out = out;
    d.odt = DT_F32;
    d.out_stride = K;
    d.accumulate = 1;
    d.topk = 1;
    if (int rc = launch_route_counts(expert_count, token_sorted, static_cast<const uint16_t*>(weight_sorted), (int)B,
                                     r, stream))
        return rc_launch(rc);
    return rc_launch(launch_decode(d, p.rmax, stream, 7));
}

int mi355moe_fp8_quant_rows(const void* x, int x_dtype, int64_t rows, int64_t K, int64_t x_stride, void* q,
                            float* scale, hipStream_t stream) {
    if (!x || !q || !scale) return MI355MOE_EINVAL;
    if (dt_w(x_dtype) < 0) return MI355MOE_EDTYPE;
    if (rows < 0 || rows > (1 << 30) || K < 4 || K % 4 || x_stride < K) return MI355MOE_ESHAPE;
    return rc_launch(launch_quant_rows(x, dt_w(x_dtype), x_stride, (int)rows, (int)K, static_cast<uint8_t*>(q), scale,
                                       stream));
}

int64_t mi355moe_fp8_moe_workspace_bytes(const mi355moe_fp8_layer* layer, int64_t T, int64_t topk) {
    if (fp8_layer_ok(layer) || T < 0 || topk < 1 || topk > MAX_TOPK) return -1;
    const int64_t P = std::max<int64_t>(1, T * topk);
    Fp8Ws w;
    int sc;
    carve_fp8(nullptr, P, std::max<int64_t>(1, T), layer->n, layer->hidden, layer->intermediate, w, sc);
    return (int64_t)w.bytes;
}

int mi355moe_fp8_moe_forward_ids(const mi355moe_fp8_layer* layer, const void* x, int x_dtype, int64_t x_stride,
                                 int64_t T, const void* ids, int ids_dtype, const void* weights, int weights_dtype,
                                 int64_t topk, const int64_t* expert_map, int64_t n_global, float limit, void* out,
                                 int out_dtype, int64_t out_stride, void* workspace, size_t workspace_bytes,
                                 int stages, hipStream_t stream) {
    if (int r = fp8_layer_ok(layer)) return r;
    if (!x || !ids || !weights || !out || !workspace) return MI355MOE_EINVAL;
    if (stages <= 0 || stages > MI355MOE_STAGE_ALL) return MI355MOE_EINVAL;
    if (dt_w(x_dtype) < 0 || dt_w(weights_dtype) < 0 || dt_w(out_dtype) < 0) return MI355MOE_EDTYPE;
    if (ids_dtype != MI355MOE_I32 && ids_dtype != MI355MOE_I64) return MI355MOE_EDTYPE;
    const int64_t K = layer->hidden, N = layer->intermediate, n = layer->n;
    if (T < 0 || topk < 1 || topk > MAX_TOPK) return MI355MOE_ELIMIT;
    if (x_stride < K || out_stride < K || out_stride % 2) return MI355MOE_ESHAPE;
    if (expert_map && n_global < 0) return MI355MOE_EINVAL;
    const int64_t P = T * topk;
    if (P > MAX_PAIRS) return MI355MOE_ELIMIT;
    if (T == 0) return 0;
    Fp8Ws w;
    int S_cap;
    carve_fp8(workspace, P, T, n, K, N, w, S_cap);
    if (workspace_bytes < w.bytes) return MI355MOE_EWORKSPACE;
    if (S_cap > 65535) return MI355MOE_ELIMIT;
    RouteArgs& r = w.ra;
    r.ids = ids;
    r.ids64 = ids_dtype == MI355MOE_I64;
    r.w = weights;
    r.wdt = dt_w(weights_dtype);
    r.emap = expert_map;
    r.n_global = expert_map ? n_global : 0;
    r.P = (int)P;
    r.topk = (int)topk;
    r.n = (int)n;
    r.R = 1 << 30;
    r.seg = FP8_TM;
    r.S_cap = S_cap;
    Fp8Args& f = w.fa;
    f.n = (int)n;
    f.K = (int)K;
    f.N = (int)N;
    f.P = (int)P;
    f.T = (int)T;
    f.w13 = static_cast<const uint8_t*>(layer->w13);
    f.w13s = layer->w13_scale;
    f.w2 = static_cast<const uint8_t*>(layer->w2);
    f.w2s = layer->w2_scale;
    f.x = x;
    f.xdt = dt_w(x_dtype);
    f.x_stride = x_stride;
    f.tok = r.tok;
    f.w32 = r.w32;
    f.pe = r.pe;
    f.inv = r.inv;
    f.topk = (int)topk;
    f.seg_expert = r.seg_expert;
    f.seg_row0 = r.seg_row0;
    f.seg_rows = r.seg_rows;
    f.nseg = r.nseg;
    f.S_cap = S_cap;
    f.limit = limit;
    f.out = out;
    f.odt = dt_w(out_dtype);
    f.out_stride = out_stride;
    int kernels = 0;
    if (stages & MI355MOE_STAGE_ROUTE) {
        if (int rc = launch_route(r, stream)) return rc_launch(rc);
        kernels |= 1;
    }
    if (stages & MI355MOE_STAGE_GATEUP) kernels |= 2;
    if (stages & MI355MOE_STAGE_DOWN) kernels |= 4;
    if (stages & MI355MOE_STAGE_COMBINE) kernels |= 8;
    return rc_launch(launch_fp8(f, stream, kernels));
}

}  // extern "C"

