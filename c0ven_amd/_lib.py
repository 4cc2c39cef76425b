"""ctypes bindings of include/c0ven_moe.h (libc0ven_moe.so, built in-tree by __graft_entry__.build()).

There is no fallback: importing this module without the built library raises, and every compute call goes to the
HIP library.
"""
import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libc0ven_moe.so")

if not os.path.exists(LIB_PATH):
    raise ImportError("c0ven_amd: %s is not built; run __graft_entry__.build()" % LIB_PATH)
lib = C.CDLL(LIB_PATH)

QT_Q8_0, QT_Q4_K, QT_Q8_K, QT_IQ3_XXS, QT_IQ4_NL, QT_IQ3_S, QT_IQ2_S, QT_Q2_0 = 8, 12, 15, 18, 20, 21, 22, 42
QT_Q5_K, QT_Q6_K, QT_IQ4_XS = 13, 14, 23
TYPE_NAMES = {QT_Q8_0: "Q8_0", QT_Q4_K: "Q4_K", QT_Q5_K: "Q5_K", QT_Q6_K: "Q6_K", QT_IQ3_S: "IQ3_S",
              QT_IQ4_NL: "IQ4_NL", QT_IQ4_XS: "IQ4_XS", QT_Q2_0: "Q2_0", QT_IQ3_XXS: "IQ3_XXS", QT_IQ2_S: "IQ2_S"}
TYPE_IDS = {v: k for k, v in TYPE_NAMES.items()}
BLOCK = {QT_Q8_0: (32, 34), QT_Q4_K: (256, 144), QT_Q5_K: (256, 176), QT_Q6_K: (256, 210), QT_IQ3_S: (256, 110),
         QT_IQ4_NL: (32, 18), QT_IQ4_XS: (256, 136), QT_Q2_0: (64, 18), QT_IQ3_XXS: (256, 98), QT_IQ2_S: (256, 82)}
CODEBOOK_TYPES = (QT_IQ3_XXS, QT_IQ2_S)  # decoded through the caller's codebooks (set_codebooks)
# The codebook buffer's layout (c0ven_quant.h QGRID_*): byte offsets of iq2s_grid, iq3xxs_grid, iq3s_grid, kvalues.
QGRID_IQ2S, QGRID_IQ3XXS, QGRID_IQ3S, QGRID_KVALUES, QGRID_BYTES = 0, 8192, 9216, 11264, 33808
Q8_FAMILY = (QT_Q8_0, QT_IQ4_NL, QT_Q2_0)  # the weight types whose dot products take q8_0 activations

MOE_OK, MOE_ERROR, MOE_BAD_ARGUMENT, MOE_BUSY, MOE_TIMEOUT = 0, 1, 2, 3, 4
MOE_FLAG_EXACT_ROUTER = 1
MOE_FLAG_HC_FIXED_ORDER = 2


class MoeConfig(C.Structure):
    _fields_ = [
        ("n_embd", C.c_uint32), ("n_ff", C.c_uint32), ("n_expert", C.c_uint32), ("n_used", C.c_uint32),
        ("n_layer", C.c_uint32), ("gate_type", C.c_uint32), ("down_type", C.c_uint32), ("has_shared", C.c_uint32),
        ("sh_gate_type", C.c_uint32), ("sh_down_type", C.c_uint32), ("max_tokens", C.c_uint32),
        ("swiglu_limit", C.c_float), ("device", C.c_int32), ("borrowed_immutable", C.c_uint32),
        ("hc_lr", C.c_uint32), ("sh_up_type", C.c_uint32), ("flags", C.c_uint32),
    ]


class MoeRouteOut(C.Structure):
    _fields_ = [("ids", C.POINTER(C.c_int32)), ("w", C.POINTER(C.c_float))]


class MoeJob(C.Structure):
    _fields_ = [("layer", C.c_uint32), ("expert", C.c_uint32), ("tok", C.c_uint32), ("w", C.c_float)]


class MoeExpertWeights(C.Structure):
    _fields_ = [("gate", C.c_void_p), ("up", C.c_void_p), ("down", C.c_void_p), ("down_parts", C.c_uint32),
                ("down_blocks", C.c_uint16 * 2)]


class MoeCmJob(C.Structure):
    _fields_ = [("expert", MoeExpertWeights), ("tok", C.c_uint32), ("w", C.c_float)]


class MoeAbiRow(C.Structure):
    _fields_ = [("name", C.c_char_p), ("offset", C.c_uint32), ("size", C.c_uint32)]


class MoeTile(C.Structure):
    _fields_ = [("expert", C.c_uint32), ("slot", C.c_uint32), ("start", C.c_uint32), ("count", C.c_uint32)]


class MoeGroup(C.Structure):
    _fields_ = [("slot", C.c_int32), ("n", C.c_uint32), ("asg", C.c_uint32 * 8)]


class GgufTensorInfo(C.Structure):
    _fields_ = [("name", C.c_char_p), ("type", C.c_uint32), ("n_dims", C.c_uint32), ("shape", C.c_uint64 * 4),
                ("shard", C.c_uint32), ("offset", C.c_uint64), ("bytes", C.c_uint64), ("data", C.c_void_p)]


_P = C.c_void_p
_u32, _u64, _i32, _f32 = C.c_uint32, C.c_uint64, C.c_int32, C.c_float
_SIGS = {
    "moe_open": (_i32, [C.POINTER(MoeConfig), C.POINTER(_P)]),
    "moe_close": (None, [_P]),
    "moe_last_error": (C.c_char_p, [_P]),
    "moe_load_router": (_i32, [_P, _u32, _P, _P]),
    "moe_load_expert": (_i32, [_P, _u32, _u32, _P, _P, _P]),
    "moe_forward": (_i32, [_P, _u32, _P, _u32, _u64, _P, _u64, C.POINTER(MoeRouteOut)]),
    "moe_forward_async": (_i32, [_P, _u32, _P, _u32, _P, _P, _P, _P]),
    "moe_forward_async_noalloc": (_i32, [_P, _u32, _P, _u32, _P, _P, _P, _P]),
    "moe_compute_many": (_i32, [_P, C.POINTER(MoeCmJob), _u32, _u32, _P, _u64, _P, _u64]),
    "moe_forward_experts": (_i32, [_P, C.POINTER(MoeJob), _u32, _u32, _P, _u64, _P, _u64]),
    "moe_h_rows": (_u32, [C.POINTER(MoeConfig)]),
    "moe_check_config": (_i32, [C.POINTER(MoeConfig)]),
    "moe_prefill_dispatch": (_i32, [_P, C.POINTER(MoeTile), _u32, C.POINTER(_u32), _P]),
    "moe_prefill_exact_tokens": (_i32, [_P, C.POINTER(_u32)]),
    "moe_sync": (_i32, [_P]),
    "moe_check": (_i32, [_P, _P]),
    "moe_stream": (_P, [_P]),
    "moe_set_timing": (_i32, [_P, C.c_int]),
    "moe_kernel_times": (_i32, [_P, C.POINTER(C.c_char_p), C.POINTER(_f32), _u32, C.POINTER(_u32), C.POINTER(_u32)]),
    "moe_copy_experts": (_i32, [_P, _u32, _u32]),
    "moe_set_trace": (_i32, [_P, C.c_int]),
    "moe_trace": (_i32, [_P, _P, _u32, C.POINTER(_u32), _P]),
    "moe_grid": (_u32, [_P]),
    "moe_set_resident": (_i32, [_P, _u32, _P]),
    "moe_miss_buffers": (_i32, [_P, C.POINTER(_P), C.POINTER(_u64), C.POINTER(_P), C.POINTER(_P)]),
    "moe_last_step": (_u32, [_P]),
    "moe_set_grid": (_i32, [_P, _u32]),
    "moe_expert_bytes": (_i32, [_P, _u32, C.POINTER(_u64)]),
    "moe_device_bytes": (_u64, [_P]),
    "moe_dequantize": (_i32, [_P, _u32, _P, _u32, _u32, _P]),
    "moe_synth_normal": (None, [_u64, _u64, _f32, _P, _u64, C.c_int]),
    "moe_quantize": (_i32, [_u32, _P, _u32, _u32, _P, C.c_int]),
    "moe_synth_matrix": (_i32, [_u64, _u64, _f32, _u32, _u32, _u32, _P, C.c_int]),
    "moe_set_codebooks": (_i32, [_P, _P, _u64]),
    "moe_synth_set_codebooks": (_i32, [_P, _u64]),
    "moe_zipf_bias": (None, [_u64, _u32, _f32, _P]),
    "moe_row_bytes": (_u64, [_u32, _u32]),
    "moe_abi_layout": (_u32, [C.POINTER(MoeAbiRow), _u32]),
    "moe_load_layer_gguf": (_i32, [_P, _u32, _P, _u32]),
    "moe_load_hc": (_i32, [_P, _u32, _P, _P, _P, _P]),
    "moe_forward_hc_async": (_i32, [_P, _u32, _P, _u32, _P, _P, _P, _P]),
    "moe_forward_hc": (_i32, [_P, _u32, _P, _u32, _P, C.POINTER(MoeRouteOut)]),
    "gguf_open": (_i32, [C.c_char_p, C.POINTER(_P)]),
    "gguf_close": (None, [_P]),
    "gguf_last_error": (C.c_char_p, [_P]),
    "gguf_n_files": (_u32, [_P]),
    "gguf_n_tensors": (_u64, [_P]),
    "gguf_tensor_at": (_i32, [_P, _u64, C.POINTER(GgufTensorInfo)]),
    "gguf_find_tensor": (_i32, [_P, C.c_char_p, C.POINTER(GgufTensorInfo)]),
    "gguf_has_key": (C.c_int, [_P, C.c_char_p]),
    "gguf_get_int": (_i32, [_P, C.c_char_p, C.POINTER(C.c_int64)]),
    "gguf_get_float": (_i32, [_P, C.c_char_p, C.POINTER(C.c_double)]),
    "gguf_get_string": (_i32, [_P, C.c_char_p, C.c_char_p, _u64, C.POINTER(_u64)]),
    "gguf_get_ints": (_i32, [_P, C.c_char_p, C.POINTER(C.c_int64), _u64, C.POINTER(_u64)]),
    "gguf_architecture": (_i32, [C.c_char_p, C.c_char_p, _u64]),
    "gguf_release": (_i32, [_P, C.c_char_p, _u64, _u64]),
    "gguf_type_bytes": (_u64, [_u32, _u64]),
}
EXPORTS = tuple(_SIGS)
for _name, (_res, _args) in _SIGS.items():
    _f = getattr(lib, _name)
    _f.restype = _res
    _f.argtypes = _args


def _ptr(a):
    return a.ctypes.data_as(_P) if a is not None else None


class MoeError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__("moe status %d: %s" % (status, msg))
        self.status = status


def row_bytes(qtype, cols):
    return int(lib.moe_row_bytes(qtype, cols))


def synth_normal(seed, stream, n, sigma=1.0, nthreads=0):
    out = np.empty(n, dtype=np.float32)
    lib.moe_synth_normal(seed, stream, sigma, _ptr(out), n, nthreads)
    return out


def quantize(qtype, x, nthreads=0):
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, cols = x.shape
    out = np.empty(rows * row_bytes(qtype, cols), dtype=np.uint8)
    st = lib.moe_quantize(qtype, _ptr(x), rows, cols, _ptr(out), nthreads)
    if st != MOE_OK:
        raise MoeError(st, "moe_quantize")
    return out


def synth_matrix(seed, stream, qtype, rows, cols, sigma=0.02, nthreads=0):
    out = np.empty(rows * row_bytes(qtype, cols), dtype=np.uint8)
    st = lib.moe_synth_matrix(seed, stream, sigma, qtype, rows, cols, _ptr(out), nthreads)
    if st != MOE_OK:
        raise MoeError(st, "moe_synth_matrix")
    return out


def synth_set_codebooks(qgrid):
    """The codebooks (a QGRID-layout uint8 buffer) the IQ3_XXS and IQ2_S quantisers search."""
    qgrid = np.ascontiguousarray(qgrid, dtype=np.uint8)
    st = lib.moe_synth_set_codebooks(_ptr(qgrid), qgrid.size)
    if st != MOE_OK:
        raise MoeError(st, "moe_synth_set_codebooks")


class GgufFile:
    """A GGUF v3 model file (or its shards) mapped read-only (include/c0ven_gguf.h)."""

    def __init__(self, path):
        self.h = None
        h = _P()
        st = lib.gguf_open(path.encode(), C.byref(h))
        if st != MOE_OK:
            raise MoeError(st, lib.gguf_last_error(None).decode())
        self.h = h

    def _check(self, st):
        if st != MOE_OK:
            raise MoeError(st, lib.gguf_last_error(self.h).decode())

    def close(self):
        if self.h:
            lib.gguf_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    @property
    def n_files(self):
        return int(lib.gguf_n_files(self.h))

    @staticmethod
    def _info(t):
        return {"name": t.name.decode(), "type": t.type, "shape": tuple(t.shape[:t.n_dims]), "shard": t.shard,
                "offset": t.offset, "bytes": t.bytes, "data": t.data}

    def tensors(self):
        out = []
        for i in range(int(lib.gguf_n_tensors(self.h))):
            t = GgufTensorInfo()
            self._check(lib.gguf_tensor_at(self.h, i, C.byref(t)))
            out.append(self._info(t))
        return out

    def tensor(self, name):
        t = GgufTensorInfo()
        self._check(lib.gguf_find_tensor(self.h, name.encode(), C.byref(t)))
        return self._info(t)

    def tensor_bytes(self, name):
        """A copy of a tensor's bytes as uint8."""
        t = self.tensor(name)
        return np.ctypeslib.as_array((C.c_uint8 * t["bytes"]).from_address(t["data"])).copy()

    def has(self, key):
        return bool(lib.gguf_has_key(self.h, key.encode()))

    def get_int(self, key):
        v = C.c_int64()
        self._check(lib.gguf_get_int(self.h, key.encode(), C.byref(v)))
        return v.value

    def get_float(self, key):
        v = C.c_double()
        self._check(lib.gguf_get_float(self.h, key.encode(), C.byref(v)))
        return v.value

    def get_string(self, key):
        n = _u64()
        self._check(lib.gguf_get_string(self.h, key.encode(), None, 0, C.byref(n)))
        buf = C.create_string_buffer(n.value + 1)
        self._check(lib.gguf_get_string(self.h, key.encode(), buf, n.value + 1, C.byref(n)))
        return buf.value.decode()

    def get_ints(self, key):
        n = _u64()
        self._check(lib.gguf_get_ints(self.h, key.encode(), None, 0, C.byref(n)))
        out = (C.c_int64 * max(1, n.value))()
        self._check(lib.gguf_get_ints(self.h, key.encode(), out, n.value, C.byref(n)))
        return list(out[:n.value])

    def release(self, name, off=0, nbytes=None):
        t = self.tensor(name)
        self._check(lib.gguf_release(self.h, name.encode(), off, t["bytes"] - off if nbytes is None else nbytes))


def gguf_architecture(path):
    buf = C.create_string_buffer(256)
    st = lib.gguf_architecture(path.encode(), buf, 256)
    if st != MOE_OK:
        raise MoeError(st, lib.gguf_last_error(None).decode())
    return buf.value.decode()


def zipf_bias(seed, n_expert, s=1.1):
    out = np.empty(n_expert, dtype=np.float32)
    lib.moe_zipf_bias(seed, n_expert, s, _ptr(out))
    return out


def abi_layout():
    n = lib.moe_abi_layout(None, 0)
    rows = (MoeAbiRow * n)()
    lib.moe_abi_layout(rows, n)
    return [(r.name.decode(), r.offset, r.size) for r in rows]


class MoeBlock:
    """One context of the HIP MoE block (moe_open .. moe_close)."""

    def __init__(self, n_embd, n_ff, n_expert, n_used, gate_type, down_type, has_shared=True, sh_gate_type=None,
                 sh_down_type=None, n_layer=1, max_tokens=16, swiglu_limit=0.0, device=0, borrowed_immutable=0,
                 hc_lr=0, sh_up_type=None, exact_router=False, hc_fixed_order=False):
        self.cfg = MoeConfig(n_embd=n_embd, n_ff=n_ff, n_expert=n_expert, n_used=n_used, n_layer=n_layer,
                             gate_type=gate_type, down_type=down_type, has_shared=1 if has_shared else 0,
                             sh_gate_type=sh_gate_type if sh_gate_type is not None else gate_type,
                             sh_down_type=sh_down_type if sh_down_type is not None else down_type,
                             max_tokens=max_tokens, swiglu_limit=swiglu_limit, device=device,
                             borrowed_immutable=borrowed_immutable, hc_lr=hc_lr,
                             sh_up_type=0 if sh_up_type is None else sh_up_type,
                             flags=(MOE_FLAG_EXACT_ROUTER if exact_router else 0)
                             | (MOE_FLAG_HC_FIXED_ORDER if hc_fixed_order else 0))
        self.exact_router = bool(exact_router)
        h = _P()
        st = lib.moe_open(C.byref(self.cfg), C.byref(h))
        if st != MOE_OK:
            raise MoeError(st, lib.moe_last_error(None).decode())
        self.h = h

    def bit_exact(self, ntok):
        """Whether a forward of ntok tokens reproduces the oracle's bits (the decode kernel, or the prefill path with
        the exact router), rather than its ids with y within the tolerance."""
        return ntok <= 16 or self.exact_router

    def _check(self, st):
        if st != MOE_OK:
            raise MoeError(st, lib.moe_last_error(self.h).decode())

    def close(self):
        if self.h:
            lib.moe_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def load_router(self, layer, router_bf16, bias=None):
        r = np.ascontiguousarray(router_bf16, dtype=np.uint16)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        self._check(lib.moe_load_router(self.h, layer, _ptr(r), _ptr(b)))

    def load_expert(self, layer, expert, gate, up, down):
        self._check(lib.moe_load_expert(self.h, layer, expert, _ptr(gate), _ptr(up), _ptr(down)))

    def forward(self, layer, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        T, H = x.shape
        y = np.empty((T, H), dtype=np.float32)
        K = self.cfg.n_used
        ids = np.empty((T, K), dtype=np.int32)
        w = np.empty((T, K), dtype=np.float32)
        ro = MoeRouteOut(ids.ctypes.data_as(C.POINTER(C.c_int32)), w.ctypes.data_as(C.POINTER(C.c_float)))
        self._check(lib.moe_forward(self.h, layer, _ptr(x), T, H, _ptr(y), H, C.byref(ro)))
        return y, ids, w

    def load_hc(self, layer, gamma, w_down, w_inject, w_up):
        """The layer's hyper-connection module: gamma (4 H fp32), W_down (lr x 4H), W_inject (4 x 4H), W_up (4H x lr)
        as bf16 bits (uint16)."""
        args = [np.ascontiguousarray(gamma, dtype=np.float32)] + [np.ascontiguousarray(a, dtype=np.uint16)
                                                                  for a in (w_down, w_inject, w_up)]
        self._check(lib.moe_load_hc(self.h, layer, *[_ptr(a) for a in args]))

    def forward_hc(self, layer, R):
        """The block with its hyper-connection mix and combine: R (T x 4 x H) in; R updated, y, ids, w out."""
        R = np.array(R, dtype=np.float32, copy=True, order="C")
        T = R.shape[0]
        H, K = self.cfg.n_embd, self.cfg.n_used
        y = np.empty((T, H), dtype=np.float32)
        ids = np.empty((T, K), dtype=np.int32)
        w = np.empty((T, K), dtype=np.float32)
        ro = MoeRouteOut(ids.ctypes.data_as(C.POINTER(C.c_int32)), w.ctypes.data_as(C.POINTER(C.c_float)))
        self._check(lib.moe_forward_hc(self.h, layer, _ptr(R), T, _ptr(y), C.byref(ro)))
        return R, y, ids, w

    def forward_hc_async(self, layer, R_dev, ntok, y_dev=None, ids_dev=None, w_dev=None, stream=None):
        self._check(lib.moe_forward_hc_async(self.h, layer, R_dev, ntok, y_dev, ids_dev, w_dev, stream))

    def forward_async(self, layer, x_dev, ntok, y_dev, ids_dev=None, w_dev=None, stream=None):
        self._check(lib.moe_forward_async(self.h, layer, x_dev, ntok, y_dev, ids_dev, w_dev, stream))

    def forward_async_noalloc(self, layer, x_dev, ntok, y_dev, ids_dev=None, w_dev=None, stream=None):
        self._check(lib.moe_forward_async_noalloc(self.h, layer, x_dev, ntok, y_dev, ids_dev, w_dev, stream))

    def forward_experts(self, jobs, x):
        """jobs: list of (layer, expert, tok, w)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        T, H = x.shape
        arr = (MoeJob * max(1, len(jobs)))(*[MoeJob(*j) for j in jobs])
        y = np.empty((T, H), dtype=np.float32)
        self._check(lib.moe_forward_experts(self.h, arr, len(jobs), T, _ptr(x), H, _ptr(y), H))
        return y

    def compute_many(self, jobs, x):
        """jobs: list of ((gate, up, down), tok, w) or ((gate, up, down, down_parts, (b0, b1)), tok, w) with the
        matrices as uint8 arrays in the file's layout (borrowed for the call)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        T, H = x.shape
        arr = (MoeCmJob * max(1, len(jobs)))()
        for i, (m, tok, w) in enumerate(jobs):
            parts, blocks = (m[3], m[4]) if len(m) > 3 else (1, (0, 0))
            arr[i].expert = MoeExpertWeights(m[0].ctypes.data, m[1].ctypes.data, m[2].ctypes.data, parts,
                                             (C.c_uint16 * 2)(*blocks))
            arr[i].tok, arr[i].w = tok, w
        y = np.empty((T, H), dtype=np.float32)
        self._check(lib.moe_compute_many(self.h, arr, len(jobs), T, _ptr(x), H, _ptr(y), H))
        return y

    def dequantize(self, qtype, blocks, rows, cols):
        out = np.empty((rows, cols), dtype=np.float32)
        self._check(lib.moe_dequantize(self.h, qtype, _ptr(blocks), rows, cols, _ptr(out)))
        return out

    def prefill_exact_tokens(self):
        """Tokens whose top k the prefill router summed exactly since the last call."""
        n = _u32()
        self._check(lib.moe_prefill_exact_tokens(self.h, C.byref(n)))
        return n.value

    def set_resident(self, layer, resident=None):
        """Which routed experts of layer the device holds (n_expert flags; None: all)."""
        r = None if resident is None else np.ascontiguousarray(resident, dtype=np.uint8)
        self._check(lib.moe_set_resident(self.h, layer, _ptr(r)))

    def miss_buffers(self):
        """(jobs, job_stride, ans_y, ans_seq): host addresses of the hybrid's records and answer (moe_miss_buffers)."""
        j, a, q = _P(), _P(), _P()
        st = _u64()
        self._check(lib.moe_miss_buffers(self.h, C.byref(j), C.byref(st), C.byref(a), C.byref(q)))
        return j.value, st.value, a.value, q.value

    def last_step(self):
        return int(lib.moe_last_step(self.h))

    def load_layer_gguf(self, layer, gguf, blk):
        """Block blk's router and experts from a GgufFile into layer."""
        self._check(lib.moe_load_layer_gguf(self.h, layer, gguf.h, blk))

    def set_codebooks(self, qgrid):
        """iq2s_grid and iq3xxs_grid from a QGRID-layout uint8 buffer (its IQ3_S region must be ggml's grid)."""
        qgrid = np.ascontiguousarray(qgrid, dtype=np.uint8)
        self._check(lib.moe_set_codebooks(self.h, _ptr(qgrid), qgrid.size))

    def sync(self):
        self._check(lib.moe_sync(self.h))

    def check(self, stream=None):
        """Waits for stream (default: the context's) and raises MoeError (MOE_TIMEOUT) if a forward's internal wait
        gave up since the last check."""
        self._check(lib.moe_check(self.h, stream))

    def stream(self):
        return lib.moe_stream(self.h)

    def set_timing(self, on):
        """on: False, True (every kernel) or 2 (only the decode kernel and the prefill gate/up launches)."""
        self._check(lib.moe_set_timing(self.h, 2 if on == 2 else 1 if on else 0))

    def kernel_times(self):
        """{kernel: average ms per launch} over the forwards timed since timing was set (and clears them), and the
        number of forwards."""
        cap = 32
        names = (C.c_char_p * cap)()
        ms = (C.c_float * cap)()
        n, nf = C.c_uint32(), C.c_uint32()
        self._check(lib.moe_kernel_times(self.h, names, ms, cap, C.byref(n), C.byref(nf)))
        return {names[i].decode(): ms[i] for i in range(min(n.value, cap))}, nf.value

    def set_trace(self, on):
        self._check(lib.moe_set_trace(self.h, 1 if on else 0))

    def trace(self):
        """The last forward's (start, ready, computed, end) s_memrealtime stamps (100 MHz) per work item, and where
        the lead (router), top-k, shared gate/up, shared down, gate/up, down and combine items begin (plus the end)."""
        n = C.c_uint32()
        bounds = np.zeros(8, dtype=np.uint32)
        self._check(lib.moe_trace(self.h, None, 0, C.byref(n), _ptr(bounds)))
        out = np.zeros((n.value, 4), dtype=np.uint64)
        self._check(lib.moe_trace(self.h, _ptr(out), n.value, C.byref(n), _ptr(bounds)))
        return out, bounds

    def prefill_dispatch(self, ntok):
        """The last prefill forward's MoeTiles (expert, slot, start, count) and perm (row -> assignment)."""
        n = C.c_uint32()
        self._check(lib.moe_prefill_dispatch(self.h, None, 0, C.byref(n), None))
        tiles = (MoeTile * max(1, n.value))()
        perm = np.empty(ntok * self.cfg.n_used, dtype=np.uint32)
        self._check(lib.moe_prefill_dispatch(self.h, tiles, n.value, C.byref(n), _ptr(perm)))
        t = np.array([(x.expert, x.slot, x.start, x.count) for x in tiles[:n.value]], dtype=np.uint32).reshape(-1, 4)
        return t, perm

    def grid(self):
        return int(lib.moe_grid(self.h))

    def copy_experts(self, src_layer, dst_layer):
        self._check(lib.moe_copy_experts(self.h, src_layer, dst_layer))

    def expert_bytes(self, which):
        v = C.c_uint64()
        self._check(lib.moe_expert_bytes(self.h, which, C.byref(v)))
        return v.value

    def device_bytes(self):
        return int(lib.moe_device_bytes(self.h))
