"""The committed golden fixtures agree with the oracle and with the workload recipes (CPU only)."""

from pathlib import Path

import numpy as np
import torch

from mamformer_amd import workloads as W
from oracle import kda, ssd
from tests.conftest import rel_l2

GOLD = Path(__file__).resolve().parent / "golden"


def test_ssd1_fixture_is_the_workload_and_the_oracle():
    z = np.load(GOLD / "ssd1.npz")
    inp = W.ssd_inputs(W.SSD1)
    for k in ("x", "dt", "A", "B", "C", "D"):
        assert np.array_equal(z[k], inp[k].numpy()), k
    y, fin = ssd.ssd_chunked(z["x"], z["dt"], z["A"], z["B"], z["C"], z["D"], chunk_size=64)
    assert rel_l2(y, z["y"]) < 1e-6
    assert rel_l2(fin, z["final"]) < 1e-6


def test_ssd_edge_fixtures_match_direct_form():
    z = np.load(GOLD / "ssd_edge.npz")
    names = sorted({k.split("/")[0] for k in z.files})
    assert len(names) >= 6
    for n in names:
        s0 = z[f"{n}/initial_state"] if f"{n}/initial_state" in z.files else None
        y, fin = ssd.ssd_direct(z[f"{n}/x"], z[f"{n}/dt"], z[f"{n}/A"], z[f"{n}/B"], z[f"{n}/C"], z[f"{n}/D"],
                                initial_state=s0)
        assert rel_l2(y, z[f"{n}/y"]) < 1e-6, n
        assert rel_l2(fin, z[f"{n}/final"]) < 1e-6, n


def test_decode_fixture_matches_direct_update():
    z = np.load(GOLD / "decode_small.npz")
    s = z["state0"].astype(np.float64)
    for i in range(z["x"].shape[0]):
        y, s = ssd.state_update_direct(s, z["x"][i], z["dt"][i], z["A"], z["B"][i], z["C"][i], z["D"],
                                       dt_bias=z["dt_bias"], dt_softplus=True)
        assert rel_l2(y, z["y"][i]) < 1e-6
    assert rel_l2(s, z["state"]) < 1e-6


def test_kda_fixture_matches_closed_form():
    z = np.load(GOLD / "kda_small.npz")
    o, ST = kda.gated_chunked(z["q1"], z["q2"], z["k"], z["v"], z["g"], float(z["lam"]), z["S0"], chunk_size=16)
    assert rel_l2(o, z["o"]) < 1e-6
    assert rel_l2(ST, z["final"]) < 1e-6


def test_workload_recipes_are_seeded_and_shaped():
    a = W.ssd_inputs(W.SSD2.scaled(seqlen=64))
    b = W.ssd_inputs(W.SSD2.scaled(seqlen=64))
    assert torch.equal(a["x"], b["x"]) and a["x"].dtype == torch.bfloat16
    assert a["x"].shape == (2, 64, 64, 64) and a["B"].shape == (2, 64, 1, 128)
    assert float(a["A"].max()) <= -1.0 + 1e-6 and float(a["A"].min()) >= -16.0 - 1e-4
    d = W.decode_inputs(W.DEC3.scaled(batch=2))
    assert d["state"].shape == (2, 64, 64, 128) and d["dt_bias"][0] == W.DT_BIAS
    k = W.kda_inputs(W.KDA5.scaled(seqlen=16, batch=1))
    assert k["g"].max() <= 0 and k["q1"].shape == (1, 32, 16, 128)
