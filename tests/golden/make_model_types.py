"""Writes tests/golden/model_layer_types.json: the MoE tensors' types and shapes of every block of the reference's
model file, read from the reference's census docs/model/tensors-IQ3_S.tsv (a data file: name, type, ggml type,
shape, bytes, shard, offset, category). Run in a checkout that has the reference at /root/reference; the GPU box and
the tests read only the JSON it writes."""
import collections
import json
import os
import sys

SRC = "/root/reference/docs/model/tensors-IQ3_S.tsv"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "model_layer_types.json")
KEYS = ["ffn_gate_exps", "ffn_up_exps", "ffn_down_exps", "ffn_gate_shexp", "ffn_up_shexp", "ffn_down_shexp",
        "ffn_gate_inp", "ffn_gate_inp_shexp"]


def main(src=SRC):
    layers = collections.defaultdict(dict)
    with open(src) as f:
        next(f)
        for line in f:
            name, tname, tid, shape = line.rstrip("\n").split("\t")[:4]
            parts = name.split(".")
            if parts[0] != "blk" or parts[2] not in KEYS:
                continue
            layers[int(parts[1])][parts[2]] = {"type": tname, "ggml_type": int(tid),
                                               "shape": [int(v) for v in shape.split("x")]}
    out = {"source": "docs/model/tensors-IQ3_S.tsv", "layers": [layers[b] for b in sorted(layers)]}
    with open(OUT, "w") as f:
        json.dump(out, f, sort_keys=True, separators=(",", ":"))
    print("wrote", OUT, len(out["layers"]), "layers")


if __name__ == "__main__":
    main(*sys.argv[1:])
