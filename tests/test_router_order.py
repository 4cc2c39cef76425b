"""Two summation orders the router's parity rests on, measured on the CPU at BASELINE config 2's router (H 2048,
512 experts + the shared gate, top-10, N(0, 0.02) bf16 weights, N(0, 1) tokens, Zipf(1.1) logit bias).

1. Router logits. The oracle (and both GPU paths) round the exact fp64 sum of the bf16 products once to fp32. ggml's
   BF16 vec_dot accumulates in fp32 instead (SIMD partial sums, then a reduction), which the reference does not
   restate. This measures how often an fp32-accumulating dot (32 partial sums, each adding its exact products in
   sequence, then a pairwise reduction) changes the top-10 set or its order against the exactly rounded logits.
2. The softmax's double sum. The oracle adds expf(l_e - max) in expert order; the GPU adds per-lane partials (lane l:
   experts l, l + 64, ...) and reduces them over the wave (prefill: one sum; decode: three parts, each reduced, then
   added). A double sum of floats is exact only while the terms' exponents stay within ~29 bits of each other, so
   1 / sum can differ in the last place. This counts how often (float)(1 / sum) differs between the orders.

Both are reported (printed, and recorded in the design notes) and bounded here, so that a change that makes either
rate grow fails.
"""
import numpy as np

from tests import harness as h
from tests.harness import moe

H, E, K = 2048, 512, 10
NTOK = 10240


def _router():
    L = h.Layer(H, 256, E, K, moe.QT_Q8_0, moe.QT_Q8_0, seed=2026, zipf=1.1, experts=[], has_shared=False)
    W = h.bf16_to_f32(L.router).astype(np.float64)  # (E + 1) x H
    return L, W


def _fp32_lane_dot(w, x, lanes=32):
    """sum_i w_i x_i with fp32 partial sums: lane j adds the exact products i = j, j + lanes, ... in sequence; then
    the lanes are added pairwise."""
    p = (w.astype(np.float32) * x.astype(np.float32)).reshape(-1, H // lanes, lanes)  # exact: bf16 x bf16
    acc = np.zeros((p.shape[0], lanes), np.float32)
    for s in range(H // lanes):
        acc = acc + p[:, s, :]
    while acc.shape[1] > 1:
        acc = acc[:, 0::2] + acc[:, 1::2]
    return acc[:, 0]


def _topk(lg, k):
    # larger first, ties to the lower id (a stable sort of the negated logits)
    return np.argsort(-lg, kind="stable")[:k]


def test_router_fp32_accumulation_rate():
    L, W = _router()
    x = h.tokens(77, NTOK, H)
    xb = h.bf16_to_f32(h.to_bf16(x)).astype(np.float64)
    lg64 = (xb @ W[:E].T).astype(np.float32) + L.bias  # exactly rounded up to fp64 summation error (~1e-16)
    # Only tokens with two of their top-11 logits closer than the fp32 accumulation error bound can change.
    s = -np.sort(-lg64, axis=1)[:, :K + 1]
    gaps = np.min(s[:, :-1] - s[:, 1:], axis=1)
    bound = 64 * 6e-8 * np.abs(xb) @ np.abs(W[:E]).max(axis=0)  # sequential fp32 error bound per token (loose)
    near = np.nonzero(gaps < bound)[0]
    set_changes = order_changes = 0
    for t in near:
        lg32 = _fp32_lane_dot(W[:E], np.broadcast_to(xb[t], (E, H))) + L.bias
        a, b = _topk(lg64[t], K), _topk(lg32, K)
        if set(a.tolist()) != set(b.tolist()):
            set_changes += 1
        elif not np.array_equal(a, b):
            order_changes += 1
    print("router fp32 accumulation: %d tokens, %d near ties checked, top-10 set changed %d, order only %d"
          % (NTOK, len(near), set_changes, order_changes))
    assert (set_changes + order_changes) / NTOK < 0.01


def _gpu_wave_sum(v):
    """wave_sum_f64 (device_math.h) over 64 lane values: xor-1, xor-2, half-mirror (8-lane rows reversed), mirror
    (16-lane rows reversed) DPP steps, then the four row totals added as (r0 + r1) + (r2 + r3)."""
    v = np.asarray(v, np.float64).copy()
    idx = np.arange(64)
    for perm in (idx ^ 1, idx ^ 2, (idx & ~7) | (7 - (idx & 7)), (idx & ~15) | (15 - (idx & 15))):
        v = v + v[perm]
    return (v[0] + v[16]) + (v[32] + v[48])


def test_softmax_sum_order_rate():
    L, W = _router()
    n = 4096
    x = h.tokens(78, n, H)
    lg, _, _ = L.oracle_route(x[:n])
    lg = lg[:, :E]
    mx = lg.max(axis=1, keepdims=True)
    ex = h.orc_expf((lg - mx).astype(np.float32).ravel()).reshape(n, E).astype(np.float64)
    diff_pf = diff_dec = 0
    for t in range(n):
        e = ex[t]
        ref = 0.0
        for v in e:
            ref += v
        lanes = e.reshape(8, 64)  # lane l holds experts l + 64 i
        part = np.zeros(64)
        for i in range(8):
            part = part + lanes[i]
        pf = _gpu_wave_sum(part)
        parts = []
        for p in range(3):  # the decode kernel's three parts: slots i = p, p + 3, ...
            acc = np.zeros(64)
            for i in range(p, 8, 3):
                acc = acc + lanes[i]
            parts.append(_gpu_wave_sum(acc))
        dec = (parts[0] + parts[1]) + parts[2]
        f = lambda s: np.float32(1.0 / s)
        diff_pf += f(pf) != f(ref)
        diff_dec += f(dec) != f(ref)
    print("softmax double sum: %d tokens, (float)(1/sum) differs from expert order: prefill order %d, decode order %d"
          % (n, diff_pf, diff_dec))
    assert diff_pf / n < 0.001 and diff_dec / n < 0.001
