"""The compiler's resource figures for the hot kernels, as the last build() recorded them: the decode kernel is
persistent (its grid is what the device holds at once), so a spill or a lost wave a SIMD costs every forward; the
prefill GEMMs are sized for their occupancy too. Skipped when no build has run in this tree."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
RESOURCES = os.path.join(ROOT, "c0ven_amd", "_build", "kernel_resources.txt")


def _rows():
    if not os.path.exists(RESOURCES):
        pytest.skip("no build in this tree (run __graft_entry__.build())")
    rows = {}
    for line in open(RESOURCES):
        name, *kv = line.split()
        rows[name] = {k: int(v) if v.isdigit() else v for k, v in (x.split("=") for x in kv)}
    return rows


def test_decode_instantiations_do_not_spill():
    rows = _rows()
    dec = {n: r for n, r in rows.items() if n.startswith("_ZN5c0ven10moe_decodeI")}
    plain = {n: r for n, r in dec.items() if "ELb0EE" in n}
    assert len(plain) == 15 and len(dec) == 30, sorted(dec)
    for n, r in plain.items():
        assert r["scratch"] == 0, (n, r)
        assert r["occupancy"] >= 3, (n, r)
    for n, r in dec.items():  # the hyper-connection forms: at most a few words of spill
        assert r["scratch"] <= 16 and r["occupancy"] >= 3, (n, r)


def test_prefill_kernels_do_not_spill():
    # The measured configurations' kernels (routing, dispatch, combine, quantiser; the expert GEMMs of Q4_K = 12, IQ3_S = 21 and
    # Q8_0 = 8) hold everything in registers; the other types' GEMMs may keep a few words outside the unit loop.
    rows = _rows()
    pf = {n: r for n, r in rows.items() if re.search(r"pf_(gate_up|gemm16|router|combine|quant_rows|topk|place|masks)", n)}
    assert pf
    for n, r in pf.items():
        hot = not re.search(r"pf_gemm16ILj(\d+)E", n) or re.search(r"pf_gemm16ILj(12|21|8)E", n)
        assert r["scratch"] <= (0 if hot else 16), (n, r)
