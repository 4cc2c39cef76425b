"""moe_load_layer_gguf: one block's router and experts read from a GGUF file (the names and shapes of
docs/model/tensors-IQ3_S.tsv: blk.N.ffn_gate_inp, ffn_gate_inp_shexp, ffn_{gate,up,down}_exps, ffn_*_shexp) give the
same forward as the same weights loaded call by call, checked against the oracle bit for bit; a file whose types or
shapes differ from the context's is refused."""
import sys

import numpy as np
import pytest

from tests import gguf_writer as gw
from tests import harness as h
from tests.harness import moe

pytestmark = pytest.mark.gpu


def say(*a):
    print("[gguf]", *a, flush=True)
    sys.stdout.flush()


def write_block(path, L, blk):
    pre = "blk.%d." % blk
    E, H, F = L.E, L.H, L.F
    ts = [(pre + "ffn_gate_inp.weight", 30, (H, E), L.router[:E].view(np.uint8).ravel()),
          (pre + "ffn_gate_inp_shexp.weight", 30, (H,), L.router[E].view(np.uint8).ravel()),
          (pre + "ffn_gate_exps.weight", L.gate_type, (H, F, E), np.concatenate([L.experts[e][0] for e in range(E)])),
          (pre + "ffn_up_exps.weight", L.gate_type, (H, F, E), np.concatenate([L.experts[e][1] for e in range(E)])),
          (pre + "ffn_down_exps.weight", L.down_type, (F, H, E), np.concatenate([L.experts[e][2] for e in range(E)])),
          (pre + "ffn_gate_shexp.weight", L.sh_gate_type, (H, F), L.shared[0]),
          (pre + "ffn_up_shexp.weight", L.sh_up_type, (H, F), L.shared[1]),
          (pre + "ffn_down_shexp.weight", L.sh_down_type, (F, H), L.shared[2]),
          ("output_norm.weight", 0, (H,), np.zeros(4 * H, np.uint8))]
    gw.write(path, [("general.architecture", gw.STRING, "qwen4exp"), ("qwen4exp.expert_count", gw.U32, E)], ts)


@pytest.mark.parametrize("types", [(moe.QT_IQ3_XXS, moe.QT_IQ4_NL, moe.QT_Q4_K, moe.QT_IQ4_NL, moe.QT_IQ4_XS),
                                   (moe.QT_Q4_K, moe.QT_Q8_0, moe.QT_Q8_0, moe.QT_Q8_0, moe.QT_Q8_0),
                                   (moe.QT_IQ4_XS, moe.QT_IQ4_NL, moe.QT_Q4_K, moe.QT_Q8_0, moe.QT_Q5_K)])
def test_load_layer_from_gguf(tmp_path, types):
    """(routed gate/up, routed down, shared gate, shared down, shared up): the first is the file's blk.0 (shared gate
    Q4_K, up IQ4_XS), the last its blk.47 (routed IQ4_XS, shared down Q8_0, up Q5_K)."""
    gt, dt, sgt, sdt, sut = types
    say("load_layer_gguf", [moe.TYPE_NAMES[t] for t in types])
    L = h.Layer(2560, 640, 32, 8, gt, dt, sgt, sdt, seed=31, sh_up_type=sut)
    path = str(tmp_path / "block.gguf")
    write_block(path, L, 5)
    g = moe.GgufFile(path)
    blk = L.block(n_layer=2, max_tokens=64)
    if gt in moe.CODEBOOK_TYPES:
        blk.set_codebooks(h.CODEBOOKS)
    blk.load_layer_gguf(1, g, 5)
    for T in (1, 8, 40):
        x = h.tokens(500 + T, T, 2560)
        y, ids, w = blk.forward(1, x)
        h.check_block(y, ids, w, *L.oracle_forward(x), blk.bit_exact(T))
    with pytest.raises(moe.MoeError):  # no block 4 in the file
        blk.load_layer_gguf(0, g, 4)
    blk.close()
    other = moe.MoeBlock(2560, 640, 32, 8, moe.QT_IQ3_S, dt, True, sgt, sdt, sh_up_type=sut)  # gate type differs
    with pytest.raises(moe.MoeError):
        other.load_layer_gguf(0, g, 5)
    other.close()
    other = moe.MoeBlock(2560, 640, 32, 8, gt, dt, True, sgt, sdt, sh_up_type=sgt if sut != sgt else moe.QT_IQ4_NL)
    if gt in moe.CODEBOOK_TYPES:
        other.set_codebooks(h.CODEBOOKS)
    with pytest.raises(moe.MoeError):
        other.load_layer_gguf(0, g, 5)
    other.close()
    g.close()
