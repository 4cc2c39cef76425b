"""The reference model file's MoE blocks against the block's configuration (no GPU): every one of the 48 blocks of
the IQ3_S file (tests/golden/model_layer_types.json, written from the reference's census docs/model/tensors-IQ3_S.tsv
by tests/golden/make_model_types.py) gives a moe_config that moe_check_config accepts, with the shared expert's gate,
up and down each of its own type, as the reference runs them (core/models/qwen4exp/model.cpp:828-830)."""
import json
import os

import pytest

from tests.harness import moe

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "model_layer_types.json")
LAYERS = json.load(open(GOLDEN))["layers"]


def layer_config(L):
    t = {k: v["ggml_type"] for k, v in L.items()}
    H, F, E = L["ffn_gate_exps"]["shape"]
    assert t["ffn_gate_exps"] == t["ffn_up_exps"]
    return moe.MoeConfig(n_embd=H, n_ff=F, n_expert=E, n_used=10, gate_type=t["ffn_gate_exps"],
                         down_type=t["ffn_down_exps"], has_shared=1, sh_gate_type=t["ffn_gate_shexp"],
                         sh_up_type=t["ffn_up_shexp"], sh_down_type=t["ffn_down_shexp"], max_tokens=4096)


def type_tuples():
    """The distinct (routed gate/up, routed down, shared gate, shared up, shared down) of the file."""
    seen = []
    for L in LAYERS:
        tup = tuple(L[k]["ggml_type"] for k in ("ffn_gate_exps", "ffn_down_exps", "ffn_gate_shexp", "ffn_up_shexp",
                                                   "ffn_down_shexp"))
        if tup not in seen:
            seen.append(tup)
    return seen


def test_census_shape():
    assert len(LAYERS) == 48
    assert len(type_tuples()) == 37
    for L in LAYERS:
        assert L["ffn_gate_exps"]["shape"] == [2560, 640, 512] and L["ffn_down_exps"]["shape"] == [640, 2560, 512]
        assert L["ffn_gate_shexp"]["shape"] == [2560, 640] and L["ffn_down_shexp"]["shape"] == [640, 2560]
        assert L["ffn_gate_inp"]["type"] == "BF16" and L["ffn_gate_inp"]["shape"] == [2560, 512]


@pytest.mark.parametrize("blk", range(48))
def test_every_block_is_accepted(blk):
    cfg = layer_config(LAYERS[blk])
    st = moe.lib.moe_check_config(cfg)
    assert st == moe.MOE_OK, moe.lib.moe_last_error(None).decode()


def test_mismatched_shared_activation_types_are_refused():
    cfg = layer_config(LAYERS[0])
    cfg.sh_up_type = moe.QT_Q8_0  # q8_0 activations against the gate's q8_K
    assert moe.lib.moe_check_config(cfg) == moe.MOE_BAD_ARGUMENT
    cfg = layer_config(LAYERS[0])
    cfg.sh_gate_type, cfg.sh_up_type = moe.QT_IQ3_S, moe.QT_Q4_K  # a codebook type beside another
    assert moe.lib.moe_check_config(cfg) == moe.MOE_BAD_ARGUMENT
