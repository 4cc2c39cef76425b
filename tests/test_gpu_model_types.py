"""The block on every type mix of the reference's model file (tests/golden/model_layer_types.json: the 37 distinct
(routed gate/up, routed down, shared gate, shared up, shared down) tuples of its 48 MoE blocks, at its shape n_embd
2560, n_ff 640), against the oracle bit for bit: decode (8 tokens) and prefill (100 tokens). The experts are this
library's quantisers' blocks of N(0, 0.02) weights (the file's bytes are not on this machine); IQ3_XXS and IQ2_S
decode through the tests' stand-in codebooks (ggml's tables are not here)."""
import pytest

from tests import harness as h
from tests.harness import moe
from tests.test_gpu_parity import say
from tests.test_gpu_parity import check_block
from tests.test_model_file import type_tuples

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("tup", type_tuples(), ids=lambda t: "-".join(moe.TYPE_NAMES[x] for x in t))
def test_model_file_type_mix(tup):
    gt, dt, sgt, sut, sdt = tup
    say("model types", [moe.TYPE_NAMES[t] for t in tup])
    L = h.Layer(2560, 640, 32, 8, gt, dt, sgt, sdt, seed=4700 + gt * 31 + sgt * 7 + sut, zipf=1.1, sh_up_type=sut)
    blk = L.block(max_tokens=128)
    L.upload(blk)
    for T in (8, 100):
        x = h.tokens(4800 + T, T, 2560)
        y, ids, w = blk.forward(0, x)
        check_block(y, ids, w, *L.oracle_forward(x), blk.bit_exact(T))
    blk.close()
