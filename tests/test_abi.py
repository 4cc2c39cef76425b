"""The C ABI without a GPU: the library loads, exports exactly what include/c0ven_moe.h declares, lays out its structs
as the header (and the ctypes mirror) say, and rejects bad configurations before it touches a device.

The reference's own ABI test compares struct offsets against engine_abi_layout's table (include/engine_api.h:414-421);
moe_abi_layout is that table here.
"""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

from tests import harness as h
from tests.harness import moe
from c0ven_amd import _lib

HEADERS = [os.path.join(h.ROOT, "include", f) for f in ("c0ven_moe.h", "c0ven_gguf.h")]


def declared():
    text = "".join(open(f).read() for f in HEADERS)
    return set(re.findall(r"MOE_API\s+[\w\s\*]+?\b((?:moe|gguf)_\w+)\s*\(", text))


def test_exports_match_header():
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if l.split()[-1].startswith(("moe_", "gguf_"))}
    want = declared()
    assert len(want) >= 25
    assert exported == want
    assert set(_lib.EXPORTS) == want  # the Python binding binds every entry point, with its signature
    for name in want:
        assert getattr(_lib.lib, name) is not None


def test_struct_layout_matches_ctypes():
    rows = {name: (off, size) for name, off, size in moe.abi_layout()}
    mirrors = {"moe_config": _lib.MoeConfig, "moe_route_out": _lib.MoeRouteOut, "moe_job": _lib.MoeJob,
               "MoeTile": _lib.MoeTile, "MoeGroup": _lib.MoeGroup, "moe_abi_row": _lib.MoeAbiRow,
               "moe_expert_weights": _lib.MoeExpertWeights, "moe_cm_job": _lib.MoeCmJob,
               "gguf_tensor_info": _lib.GgufTensorInfo}
    for sname, cls in mirrors.items():
        assert rows[sname] == (0, C.sizeof(cls)), sname
        for fname, _ in cls._fields_:
            f = getattr(cls, fname)
            assert rows["%s.%s" % (sname, fname)] == (f.offset, f.size), (sname, fname)
    # shared/moe_tile.h:11-33: 16 and 40 bytes
    assert rows["MoeTile"][1] == 16 and rows["MoeGroup"][1] == 40
    assert rows["MoeGroup.asg"] == (8, 32)


def test_header_constants():
    text = open(os.path.join(h.ROOT, "include", "c0ven_moe_tile.h")).read()
    assert re.search(r"#define MOE_TILE 64\b", text)
    assert re.search(r"#define MOE_GROUP_MAX 8\b", text)
    assert re.search(r"#define MOE_WG_ROWS 32\b", text)
    q = open(os.path.join(h.ROOT, "include", "c0ven_quant.h")).read()
    ids = dict(re.findall(r"#define (QT_\w+) (\d+)", q))
    # ggml's type ids, which GGUF files carry (shared/quant.h:10-40)
    assert (ids["QT_Q8_0"], ids["QT_Q4_K"], ids["QT_Q8_K"], ids["QT_IQ3_S"]) == ("8", "12", "15", "21")
    assert (moe.QT_Q8_0, moe.QT_Q4_K, moe.QT_Q8_K, moe.QT_IQ3_S) == (8, 12, 15, 21)
    # block sizes: 34 B / 32, 144 B / 256, 110 B / 256
    assert moe.row_bytes(moe.QT_Q8_0, 2048) == 64 * 34
    assert moe.row_bytes(moe.QT_Q4_K, 2048) == 8 * 144
    assert moe.row_bytes(moe.QT_IQ3_S, 2048) == 8 * 110


def cfg(**kw):
    base = dict(n_embd=2048, n_ff=512, n_expert=512, n_used=10, n_layer=1, gate_type=12, down_type=12, has_shared=1,
                sh_gate_type=12, sh_down_type=12, max_tokens=16, swiglu_limit=0.0, device=0)
    base.update(kw)
    return _lib.MoeConfig(**base)


@pytest.mark.parametrize("bad", [dict(n_embd=1000), dict(n_embd=768), dict(n_ff=384), dict(n_expert=513),
                                 dict(n_used=17), dict(n_used=0), dict(gate_type=2), dict(down_type=15),
                                 dict(sh_gate_type=30), dict(max_tokens=16385), dict(n_ff=16384),
                                 dict(swiglu_limit=-1.0)])
def test_open_rejects_bad_config_before_the_device(bad):
    out = C.c_void_p()
    st = _lib.lib.moe_open(C.byref(cfg(**bad)), C.byref(out))
    assert st == _lib.MOE_BAD_ARGUMENT
    assert not out.value
    assert len(_lib.lib.moe_last_error(None)) > 0


def test_open_null_arguments():
    assert _lib.lib.moe_open(None, None) == _lib.MOE_BAD_ARGUMENT


def test_h_rows():
    c = cfg()
    assert _lib.lib.moe_h_rows(C.byref(c)) == 256


def test_synth_is_deterministic_and_thread_count_free():
    a = moe.synth_matrix(7, 3, moe.QT_Q4_K, 64, 512, nthreads=1)
    b = moe.synth_matrix(7, 3, moe.QT_Q4_K, 64, 512, nthreads=8)
    c = moe.synth_matrix(7, 4, moe.QT_Q4_K, 64, 512, nthreads=8)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    x = moe.synth_normal(7, 3, 1 << 16, 1.0)
    assert abs(float(x.mean())) < 0.02 and abs(float(x.std()) - 1.0) < 0.02
    # synth_matrix is synth_normal then quantize
    w = moe.synth_normal(9, 1, 32 * 512, 0.02).reshape(32, 512)
    assert np.array_equal(moe.quantize(moe.QT_IQ3_S, w), moe.synth_matrix(9, 1, moe.QT_IQ3_S, 32, 512, 0.02))


@pytest.mark.parametrize("qtype, tol", [(moe.QT_Q8_0, 0.0), (moe.QT_Q4_K, 0.2), (moe.QT_IQ3_S, 0.35),
                                        (moe.QT_IQ4_NL, 0.1), (moe.QT_Q2_0, 0.5), (moe.QT_IQ3_XXS, 0.35),
                                        (moe.QT_IQ2_S, 0.45), (moe.QT_Q5_K, 0.1), (moe.QT_Q6_K, 0.06),
                                        (moe.QT_IQ4_XS, 0.15)])
def test_quantisers_write_valid_blocks(qtype, tol):
    """Q8_0 is ggml's reference rule, so each value is within half a step of its code; the others are bounded in
    relative L2 (their exact choice of codes is this library's, not ggml's search)."""
    w = moe.synth_normal(11, 2, 16 * 1024, 0.02).reshape(16, 1024)
    blocks = moe.quantize(qtype, w)
    y = h.orc_dequant(qtype, blocks, w.size).reshape(w.shape)
    if qtype == moe.QT_Q8_0:
        b = blocks.reshape(-1, 34)
        d = b[:, :2].copy().view(np.float16).astype(np.float32).ravel()
        err = np.abs(y - w).reshape(-1, 32)
        # half a step, plus what rounding d to fp16 moves the largest code (127 x half an fp16 ulp of d)
        assert np.all(err <= d[:, None] * (0.5 + 127 * 2.0 ** -11) + 1e-9)
    else:
        assert h.rel_l2(y, w) < tol


def test_zipf_bias():
    b = moe.zipf_bias(5, 512, 1.1)
    assert np.allclose(np.sort(-b / 1.1), np.log(np.arange(1, 513)), rtol=1e-6, atol=1e-6)
    p = np.exp(b) / np.exp(b).sum()
    top = np.sort(p)[::-1]
    assert top[:102].sum() > 0.6  # about a fifth of the experts take most of the mass
