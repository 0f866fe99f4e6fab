"""Router, expert map and token->expert permutation (oracle; test infrastructure only).

References:
  router     sigmoid scores, top-k of (score + e_score_correction_bias) with the lower id first among equals,
             weights = score / (sum + 1e-20) * routed_scale in pick order: code/fork/docs/ref/tf_glue.py:371-401
             (TensorFold's restatement of vLLM grouped_topk with n_group = topk_group = 1,
             code/fork/tests/router_topk_agreement.py:58-61). Logits = bf16(x @ W^T) widened to fp32
             (code/fork/docs/BF16_GEMV.md:27,38; code/fork/tests/router_topk_agreement.py:82).
             Router weights' last ulp: parity unpinned. sigmoid_f32 is the correctly rounded fp32 sigmoid (pinned
             to that definition); the reference computes 1 / (1 + exp(-x)) in fp32 with the library exp (vLLM's
             grouped_topk, not importable here; tf_glue.py:381), so its scores, and the renormalised weights built
             from them, may differ from these in the last ulp. Ids and weights are pinned by the closed form only.
  local ids  map_topk_to_local, code/fork/docs/prod_exl3_reference.py:936-958.
  order      pairs j = t*topk + k grouped by local expert, the sentinel group (id n) last, and inside a group by
             pair index -- torch.argsort(local, stable=True) (code/fork/overlay/glm53_moe_e4m3.py:462;
             code/fork/kernels/exl3.cu:742-775 computes the same stable position).
  segments   exclusive scan of the counts, eligibility 0 < c <= R, ceil(c/rows) row segments per eligible expert,
             pair_expert = -1 elsewhere: code/fork/kernels/exl3.cu:529-566 (route_prep), the torch oracle
             code/fork/tests/test_units.py:51-78; prefill tile tables code/fork/docs/prod_exl3_reference.py:1316-1361.
"""
from __future__ import annotations

import numpy as np

ROUTER_CHUNK = 512          # the router kernel's K granularity (64 lanes x 8 bf16)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> the float32 value of its bf16 rounding (RN-even)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)) << np.uint64(16)
    return r.astype(np.uint32).view(np.float32)


def router_logits(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Router logits [T, E] as production returns them: F.linear(x, W) in bf16, then .to(float32)
    (code/fork/docs/BF16_GEMV.md:27,38), i.e. the dot product rounded to bf16. Following the reference's own router
    oracle, (X.double() @ W.t()).to(bfloat16).float() (code/fork/tests/router_topk_agreement.py:82), the dot
    product of the bf16 values (given as float32 arrays) is taken in float64 -- exact for router-sized operands,
    since every product has at most 16 significant bits -- then narrowed to fp32 and to bf16, both to nearest even
    (torch narrows a double to bf16 through fp32)."""
    x = np.asarray(x, np.float32).astype(np.float64)
    w = np.asarray(w, np.float32).astype(np.float64)
    if x.shape[1] % ROUTER_CHUNK:
        raise ValueError("K must be a multiple of 512")
    return bf16_round((x @ w.T).astype(np.float32))


def sigmoid_f32(logits: np.ndarray) -> np.ndarray:
    """fp32 sigmoid, defined as the fp32 rounding of 1 / (1 + exp(-x)) evaluated in float64."""
    z = np.asarray(logits, np.float32).astype(np.float64)
    return (1.0 / (1.0 + np.exp(-z))).astype(np.float32)


def topk_sigmoid_bias(logits: np.ndarray, bias: np.ndarray, topk: int, scale: float,
                      renormalize: bool = True) -> tuple[np.ndarray, np.ndarray]:
    """ids int32 [T, topk], weights fp32 [T, topk] (tf_glue.py:371-401): score = sigmoid(logit); pick the topk
    largest score + bias, largest first, the lower id among equal values; w_k = score_k / (total + 1e-20) * scale
    with total the fp32 sum of the picked scores in pick order."""
    s = sigmoid_f32(logits)
    choice = (s + np.asarray(bias, np.float32)[None, :]).astype(np.float32)
    T, E = s.shape
    ids = np.zeros((T, topk), np.int32)
    wts = np.zeros((T, topk), np.float32)
    for t in range(T):
        c = choice[t].astype(np.float64)          # exact copies of the fp32 values
        taken = np.zeros(E, bool)
        total = np.float32(0.0)
        for k in range(topk):
            best = -1
            for e in range(E):
                if taken[e]:
                    continue
                if best < 0 or c[e] > c[best]:
                    best = e
            taken[best] = True
            ids[t, k] = best
            wts[t, k] = s[t, best]
            total = np.float32(total + s[t, best])
        if renormalize:
            denom = np.float32(total + np.float32(1e-20))
            wts[t] = (wts[t] / denom).astype(np.float32)
        wts[t] = (wts[t] * np.float32(scale)).astype(np.float32)
    return ids, wts


def map_topk_to_local(ids: np.ndarray, n_local: int, expert_map: np.ndarray | None = None) -> np.ndarray:
    """Global ids [T, topk] -> local ids [P]; invalid or non-local -> the sentinel n_local
    (prod_exl3_reference.py:936-958)."""
    flat = np.asarray(ids).reshape(-1).astype(np.int64)
    if expert_map is None:
        return np.where((flat < 0) | (flat >= n_local), n_local, flat)
    emap = np.asarray(expert_map, np.int64)
    ng = emap.size
    safe = np.clip(flat, 0, max(ng - 1, 0))
    mapped = emap[safe] if ng else np.full_like(flat, n_local)
    bad = (flat < 0) | (flat >= ng) | (mapped < 0) | (mapped >= n_local)
    return np.where(bad, n_local, mapped)


def permutation(local: np.ndarray, n: int, topk: int, R: int, seg_rows: int = 16) -> dict:
    """Stable token->expert permutation and segment tables.

    local: [P] local ids in [0, n] (n = sentinel). Returns
      counts     int64 [n + 1]   pairs per local id (last = sentinel bucket)
      order      int64 [P]       order[pos] = pair index j at sorted position pos
      inv        int32 [P]       inv[j] = pos
      token      int64 [P]       token of the pair at pos (j // topk)
      pair_expert int32 [P]      local id at pos if 0 < count <= R and id < n, else -1
      segments   (expert, row0, rows) int32 [S] each: ceil(c / seg_rows) per eligible expert, in expert order
    """
    local = np.asarray(local, np.int64)
    P = local.size
    counts = np.bincount(local, minlength=n + 1).astype(np.int64)
    order = np.argsort(local, kind="stable").astype(np.int64)
    inv = np.empty(P, np.int32)
    inv[order] = np.arange(P, dtype=np.int32)
    token = order // topk
    le = local[order]
    elig = (counts[:n] > 0) & (counts[:n] <= R)
    pe = np.where((le < n) & elig[np.minimum(le, n - 1)], le, -1).astype(np.int32)
    start = np.concatenate([[0], np.cumsum(counts[:n])[:-1]])
    se, s0, sr = [], [], []
    for e in range(n):
        c = int(counts[e])
        if not elig[e]:
            continue
        for q in range((c + seg_rows - 1) // seg_rows):
            se.append(e)
            s0.append(int(start[e]) + seg_rows * q)
            sr.append(min(seg_rows, c - seg_rows * q))
    return {"counts": counts, "order": order, "inv": inv, "token": token, "pair_expert": pe,
            "seg_expert": np.array(se, np.int32), "seg_row0": np.array(s0, np.int32),
            "seg_rows": np.array(sr, np.int32)}


def s_cap(P: int, n: int, seg_rows: int = 16) -> int:
    """Upper bound on the number of row segments (exl3.cu:908, tf_s_cap): min(P, n) + ceil(P / seg_rows)."""
    return min(P, n) + (P + seg_rows - 1) // seg_rows
