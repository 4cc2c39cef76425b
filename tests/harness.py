"""Shared test helpers: the CPU oracle's bindings (oracle/liboracle.so, the checker), synthetic layers drawn with the
library's seeded generator, and the parity metrics.

The oracle is test infrastructure: it is loaded here, by the tests, smoke() and bench.py's cpu_baseline, and by
nothing in c0ven_amd/.
"""
import ctypes as C
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import c0ven_amd as moe  # noqa: E402

ORACLE_PATH = os.path.join(ROOT, "oracle", "liboracle.so")
_P = C.c_void_p


def _load_oracle():
    if not os.path.exists(ORACLE_PATH):
        raise ImportError("oracle/liboracle.so is not built; run __graft_entry__.build()")
    o = C.CDLL(ORACLE_PATH)
    sig = {
        "orc_fp32_to_fp16": (C.c_uint16, [C.c_float]),
        "orc_fp16_to_fp32": (C.c_float, [C.c_uint16]),
        "orc_fp32_to_bf16": (C.c_uint16, [C.c_float]),
        "orc_expf": (None, [_P, _P, C.c_int64]),
        "orc_iq3s_grid": (None, [_P]),
        "orc_iq4nl_values": (None, [_P]),
        "orc_set_codebooks": (None, [_P]),
        "orc_hc_pre": (C.c_int, [_P, C.c_uint32, C.c_uint32, C.c_uint32, _P, _P, _P, _P, _P, _P]),
        "orc_hc_post": (None, [_P, C.c_uint32, C.c_uint32, _P, _P]),
        "orc_dequantize_row": (C.c_int, [C.c_uint32, _P, _P, C.c_int64]),
        "orc_quantize_act": (C.c_int, [C.c_uint32, _P, _P, C.c_int64]),
        "orc_vec_dot": (C.c_int, [C.c_uint32, C.c_int64, _P, _P, C.POINTER(C.c_float)]),
        "orc_compute_many": (C.c_int, [_P, _P, C.c_uint32, C.c_uint32, _P, C.c_uint64, _P, C.c_uint64, C.c_int]),
        "orc_compute": (C.c_int, [_P, _P, _P, _P, _P, C.c_uint32, _P, _P]),
        "orc_route": (C.c_int, [_P, _P, C.c_uint32, C.c_uint32, C.c_uint32, _P, C.c_uint32, C.c_uint64, _P, _P, _P]),
        "orc_moe_forward": (C.c_int, [_P, _P, C.c_uint32, C.c_uint64, _P, C.c_uint64, _P, _P, C.c_int]),
        "orc_fast_moe_forward": (C.c_int, [_P, _P, C.c_uint32, C.c_uint64, _P, C.c_uint64, _P, _P, C.c_int]),
        "orc_fast_isa": (C.c_char_p, []),
        "orc_moe_forward_resident": (C.c_int, [_P, _P, _P, C.c_uint32, C.c_uint64, _P, C.c_uint64, C.c_int]),
    }
    for name, (res, args) in sig.items():
        f = getattr(o, name)
        f.restype, f.argtypes = res, args
    return o


oracle = _load_oracle()


class OrcShape(C.Structure):
    _fields_ = [("gate_type", C.c_uint32), ("down_type", C.c_uint32), ("n_embd", C.c_uint32),
                ("n_ff", C.c_uint32), ("swiglu_limit", C.c_float), ("up_type", C.c_uint32)]


class OrcJob(C.Structure):
    _fields_ = [("gate", _P), ("up", _P), ("down", _P), ("tok", C.c_uint32), ("w", C.c_float)]


class OrcLayer(C.Structure):
    _fields_ = [("n_embd", C.c_uint32), ("n_ff", C.c_uint32), ("n_expert", C.c_uint32), ("n_used", C.c_uint32),
                ("gate_type", C.c_uint32), ("down_type", C.c_uint32), ("sh_gate_type", C.c_uint32),
                ("sh_down_type", C.c_uint32), ("swiglu_limit", C.c_float), ("router", _P), ("bias", _P),
                ("gate", C.POINTER(_P)), ("up", C.POINTER(_P)), ("down", C.POINTER(_P)),
                ("sh_gate", _P), ("sh_up", _P), ("sh_down", _P), ("sh_up_type", C.c_uint32)]


def ptr(a):
    return None if a is None else a.ctypes.data_as(_P)


def act_bytes(act_type, n):
    return n // 32 * 34 if act_type == moe.QT_Q8_0 else n // 256 * 292


def vec_dot_type(t):
    return moe.QT_Q8_0 if t in moe.Q8_FAMILY else moe.QT_Q8_K


def orc_dequant(qtype, blocks, n):
    out = np.empty(n, dtype=np.float32)
    assert oracle.orc_dequantize_row(qtype, ptr(blocks), ptr(out), n) == 0
    return out


def orc_quant_act(act_type, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(act_bytes(act_type, x.size), dtype=np.uint8)
    assert oracle.orc_quantize_act(act_type, ptr(x), ptr(out), x.size) == 0
    return out


def orc_vec_dot(qtype, n, w, a):
    v = C.c_float()
    assert oracle.orc_vec_dot(qtype, n, ptr(w), ptr(a), C.byref(v)) == 0
    return v.value


def orc_expf(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    oracle.orc_expf(ptr(x), ptr(y), x.size)
    return y


def orc_grid():
    g = np.empty(512, dtype=np.uint32)
    oracle.orc_iq3s_grid(ptr(g))
    return g


def orc_iq4nl():
    v = np.empty(16, dtype=np.int8)
    oracle.orc_iq4nl_values(ptr(v))
    return v


def synth_codebooks(seed=4242):
    """A QGRID-layout codebook buffer with stand-ins for ggml's iq2s_grid and iq3xxs_grid (absent here): distinct
    entries drawn from each table's byte values (8, 25, 43; 4, 12, .., 52, 62), seeded; the real iq3s_grid and
    kvalues_iq4nl in their regions. Parity against the oracle holds for any table, so the tests use this one; the
    tables' content is what only ggml-common.h could pin."""
    r = np.random.default_rng(seed)
    buf = np.zeros(moe.QGRID_BYTES, dtype=np.uint8)
    lv2 = np.array([8, 25, 43], dtype=np.uint8)
    lv3 = np.array([4, 12, 20, 28, 36, 44, 52, 62], dtype=np.uint8)
    g2 = set()
    while len(g2) < 1024:
        g2.add(bytes(lv2[r.integers(0, 3, size=8)]))
    g3 = set()
    while len(g3) < 256:
        g3.add(bytes(lv3[r.integers(0, 8, size=4)]))
    buf[moe.QGRID_IQ2S:moe.QGRID_IQ2S + 8192] = np.frombuffer(b"".join(sorted(g2)), np.uint8)
    buf[moe.QGRID_IQ3XXS:moe.QGRID_IQ3XXS + 1024] = np.frombuffer(b"".join(sorted(g3)), np.uint8)
    buf[moe.QGRID_IQ3S:moe.QGRID_IQ3S + 2048] = orc_grid().view(np.uint8)
    buf[moe.QGRID_KVALUES:moe.QGRID_KVALUES + 16] = orc_iq4nl().view(np.uint8)
    return buf


CODEBOOKS = synth_codebooks()
oracle.orc_set_codebooks(ptr(CODEBOOKS))
moe.synth_set_codebooks(CODEBOOKS)


def to_bf16(x):
    """fp32 -> bf16 bits, round to nearest even (NaN-free input)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(b):
    return (b.astype(np.uint32) << 16).view(np.float32)


class Layer:
    """A synthetic MoE layer drawn from (seed, layer): experts N(0, sigma) quantised by the library's quantisers,
    router and shared gate N(0, sigma) as bf16, optional Zipf logit bias. Expert e's matrices are streams
    layer * 2^20 + 4 e + {0, 1, 2}; the shared expert is e = n_expert."""

    def __init__(self, H, F, E, K, gate_type, down_type, sh_gate_type=None, sh_down_type=None, has_shared=True,
                 seed=1234, layer=0, sigma=0.02, zipf=None, swiglu_limit=0.0, experts=None, nthreads=0,
                 sh_up_type=None):
        self.H, self.F, self.E, self.K = H, F, E, K
        self.gate_type, self.down_type = gate_type, down_type
        self.sh_gate_type = gate_type if sh_gate_type is None else sh_gate_type
        self.sh_up_type = self.sh_gate_type if sh_up_type is None else sh_up_type
        self.sh_down_type = down_type if sh_down_type is None else sh_down_type
        self.has_shared, self.seed, self.layer, self.swiglu_limit = has_shared, seed, layer, swiglu_limit
        base = layer << 20
        r = moe.synth_normal(seed, base + 4 * (E + 1) + 3, (E + 1) * H, sigma, nthreads)
        self.router = to_bf16(r).reshape(E + 1, H)
        self.bias = None if zipf is None else moe.zipf_bias(seed * 7919 + layer, E, zipf)
        self.experts = {}
        wanted = range(E) if experts is None else experts
        for e in wanted:
            self.experts[e] = self._expert(e, gate_type, down_type, sigma, nthreads)
        self.shared = (self._expert(E, self.sh_gate_type, self.sh_down_type, sigma, nthreads, self.sh_up_type)
                       if has_shared else None)

    def _expert(self, e, gt, dt, sigma, nthreads, ut=None):
        s = (self.layer << 20) + 4 * e
        H, F = self.H, self.F
        return (moe.synth_matrix(self.seed, s, gt, F, H, sigma, nthreads),
                moe.synth_matrix(self.seed, s + 1, gt if ut is None else ut, F, H, sigma, nthreads),
                moe.synth_matrix(self.seed, s + 2, dt, H, F, sigma, nthreads))

    def upload(self, blk, layer=0):
        if {self.gate_type, self.down_type, self.sh_gate_type, self.sh_up_type, self.sh_down_type} & set(moe.CODEBOOK_TYPES):
            blk.set_codebooks(CODEBOOKS)
        blk.load_router(layer, self.router, self.bias)
        for e, (g, u, d) in self.experts.items():
            blk.load_expert(layer, e, g, u, d)
        if self.shared is not None:
            blk.load_expert(layer, self.E, *self.shared)

    def block(self, n_layer=1, max_tokens=16, device=0, exact_router=False):
        return moe.MoeBlock(self.H, self.F, self.E, self.K, self.gate_type, self.down_type, self.has_shared,
                            self.sh_gate_type, self.sh_down_type, n_layer=n_layer, max_tokens=max_tokens,
                            swiglu_limit=self.swiglu_limit, device=device, sh_up_type=self.sh_up_type,
                            exact_router=exact_router)

    def oracle_forward(self, x, nthreads=8):
        """The whole block on the CPU oracle: y, ids, w."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        T = x.shape[0]
        E = self.E
        if len(self.experts) != E:  # route first, then make sure every routed expert exists
            _, ids, _ = self.oracle_route(x)
            missing = sorted(set(int(i) for i in ids.ravel()) - set(self.experts))
            for e in missing:
                self.experts[e] = self._expert(e, self.gate_type, self.down_type, 0.02, 0)
        zero = np.zeros(1, dtype=np.uint8)
        arr = (_P * E)()
        gp, up, dp = (_P * E)(), (_P * E)(), (_P * E)()
        for e in range(E):
            g, u, d = self.experts.get(e, (zero, zero, zero))
            gp[e], up[e], dp[e] = g.ctypes.data, u.ctypes.data, d.ctypes.data
        del arr
        L = OrcLayer(self.H, self.F, E, self.K, self.gate_type, self.down_type, self.sh_gate_type, self.sh_down_type,
                     self.swiglu_limit, ptr(self.router), ptr(self.bias), gp, up, dp,
                     *(ptr(m) for m in (self.shared if self.shared is not None else (None, None, None))),
                     self.sh_up_type)
        y = np.empty((T, self.H), dtype=np.float32)
        ids = np.empty((T, self.K), dtype=np.int32)
        w = np.empty((T, self.K), dtype=np.float32)
        assert oracle.orc_moe_forward(C.byref(L), ptr(x), T, self.H, ptr(y), self.H, ptr(ids), ptr(w), nthreads) == 0
        return y, ids, w

    def _orc_layer(self):
        E = self.E
        zero = np.zeros(1, dtype=np.uint8)
        gp, up, dp = (_P * E)(), (_P * E)(), (_P * E)()
        for e in range(E):
            g, u, d = self.experts.get(e, (zero, zero, zero))
            gp[e], up[e], dp[e] = g.ctypes.data, u.ctypes.data, d.ctypes.data
        L = OrcLayer(self.H, self.F, E, self.K, self.gate_type, self.down_type, self.sh_gate_type, self.sh_down_type,
                     self.swiglu_limit, ptr(self.router), ptr(self.bias), gp, up, dp,
                     *(ptr(m) for m in (self.shared if self.shared is not None else (None, None, None))),
                     self.sh_up_type)
        return L, (gp, up, dp)

    def oracle_route(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        T = x.shape[0]
        lg = np.empty((T, self.E + 1), dtype=np.float32)
        ids = np.empty((T, self.K), dtype=np.int32)
        w = np.empty((T, self.K), dtype=np.float32)
        assert oracle.orc_route(ptr(self.router), ptr(self.bias), self.E, self.H, self.K, ptr(x), T, self.H,
                                ptr(lg), ptr(ids), ptr(w)) == 0
        return lg, ids, w


class HcModule:
    """A layer's hyper-connection module (MODEL_LAYER.md 1.1): gamma = 1 + N(0, 0.1) (the folded norm weight),
    W_down, W_inject, W_up N(0, sigma) as bf16 bits, drawn from (seed, layer)."""

    def __init__(self, H, lr, seed=5, layer=0, sigma=0.02):
        self.H, self.lr = H, lr
        base = (layer << 20) + (1 << 19)
        D = 4 * H
        self.gamma = (1.0 + moe.synth_normal(seed, base, D, 0.1)).astype(np.float32)
        self.down = to_bf16(moe.synth_normal(seed, base + 1, lr * D, sigma)).reshape(lr, D)
        self.inj = to_bf16(moe.synth_normal(seed, base + 2, 4 * D, sigma)).reshape(4, D)
        self.up = to_bf16(moe.synth_normal(seed, base + 3, D * lr, sigma)).reshape(D, lr)

    def load(self, blk, layer=0):
        blk.load_hc(layer, self.gamma, self.down, self.inj, self.up)

    def pre(self, R):
        """The oracle's mix: x (T x H) and the inject logits (T x 4)."""
        R = np.ascontiguousarray(R, dtype=np.float32)
        T = R.shape[0]
        x = np.empty((T, self.H), np.float32)
        inj = np.empty((T, 4), np.float32)
        assert oracle.orc_hc_pre(ptr(R), T, self.H, self.lr, ptr(self.gamma), ptr(self.down), ptr(self.inj),
                                 ptr(self.up), ptr(x), ptr(inj)) == 0
        return x, inj

    @staticmethod
    def post(R, inj, y):
        """The oracle's combine: R_s + 2 sigma(inject_s / 4) y, as a new array."""
        R = np.array(R, dtype=np.float32, copy=True, order="C")
        oracle.orc_hc_post(ptr(R), R.shape[0], R.shape[2], ptr(np.ascontiguousarray(inj, np.float32)),
                           ptr(np.ascontiguousarray(y, np.float32)))
        return R


def fast_forward(layer, x, nthreads=8):
    """The CPU baseline (oracle/cpu_fast.c): the block with the oracle's bits, SIMD inside. All experts must exist."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = x.shape[0]
    L, keep = layer._orc_layer()
    y = np.empty((T, layer.H), dtype=np.float32)
    ids = np.empty((T, layer.K), dtype=np.int32)
    w = np.empty((T, layer.K), dtype=np.float32)
    assert oracle.orc_fast_moe_forward(C.byref(L), ptr(x), T, layer.H, ptr(y), layer.H, ptr(ids), ptr(w), nthreads) == 0
    del keep
    return y, ids, w


def orc_compute_many(gate_type, down_type, H, F, jobs, x, swiglu_limit=0.0, nthreads=8):
    """jobs: list of ((gate, up, down), tok, w)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = x.shape[0]
    arr = (OrcJob * max(1, len(jobs)))(*[OrcJob(ptr(m[0]), ptr(m[1]), ptr(m[2]), t, w) for m, t, w in jobs])
    s = OrcShape(gate_type, down_type, H, F, swiglu_limit)
    y = np.full((T, H), np.nan, dtype=np.float32)
    assert oracle.orc_compute_many(C.byref(s), arr, len(jobs), T, ptr(x), H, ptr(y), H, nthreads) == 0
    return y


def rel_l2(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def max_abs(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


# The block's bar (north_star): top-k ids bit-exact, y within max-abs 1e-3 and rel-L2 1e-4. The prefill path's
# default router gives the oracle's ids with logits within ~1e-6 of its own, so its weights are held to W_TOL.
TOL_ABS, TOL_REL, W_TOL = 1e-3, 1e-4, 2e-5


def check_block(y, ids, w, yo, io, wo, exact=True):
    """ids equal; y within the tolerance; with exact, w and y equal bit for bit, else w within W_TOL."""
    assert np.array_equal(ids, io), "top-k ids differ"
    ma, rl = max_abs(y, yo), rel_l2(y, yo)
    assert ma <= TOL_ABS and rl <= TOL_REL, (ma, rl)
    if exact:
        assert np.array_equal(w, wo), "routing weights not bit-exact: max %g" % max_abs(w, wo)
        assert np.array_equal(y, yo), "y not bit-exact: max-abs %g rel-L2 %g" % (ma, rl)
    else:
        assert max_abs(w, wo) <= W_TOL, max_abs(w, wo)


class Dev:
    """Device buffers through the HIP runtime (ctypes)."""

    def __init__(self):
        self.rt = C.CDLL("libamdhip64.so")
        self.rt.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        self.rt.hipFree.argtypes = [C.c_void_p]
        self.rt.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        self.bufs = []

    def alloc(self, n):
        p = C.c_void_p()
        assert self.rt.hipMalloc(C.byref(p), max(n, 256)) == 0
        self.bufs.append(p)
        return p

    def put(self, a):
        p = self.alloc(a.nbytes)
        assert self.rt.hipMemcpy(p, a.ctypes.data_as(C.c_void_p), a.nbytes, 1) == 0
        return p

    def get(self, p, shape, dtype):
        a = np.empty(shape, dtype)
        assert self.rt.hipMemcpy(a.ctypes.data_as(C.c_void_p), p, a.nbytes, 2) == 0
        return a

    def free(self):
        for p in self.bufs:
            self.rt.hipFree(p)
        self.bufs = []


def tokens(seed, T, H, stream=999):
    return moe.synth_normal(seed, stream, T * H, 1.0).reshape(T, H)


def smoke_check():
    """One small forward on cuda:0 against the oracle (used by __graft_entry__.smoke)."""
    L = Layer(512, 256, 32, 4, moe.QT_Q4_K, moe.QT_Q8_0, seed=7)
    blk = L.block()
    L.upload(blk)
    x = tokens(7, 2, 512)
    y, ids, w = blk.forward(0, x)
    yo, io, wo = L.oracle_forward(x)
    assert np.array_equal(ids, io), (ids, io)
    assert max_abs(y, yo) <= 1e-3 and rel_l2(y, yo) <= 1e-4, (max_abs(y, yo), rel_l2(y, yo))
    blk.close()
    print("smoke ok: max_abs %.3g rel_l2 %.3g, ids equal, y bit-exact: %s" % (max_abs(y, yo), rel_l2(y, yo),
                                                                             np.array_equal(y, yo)))
