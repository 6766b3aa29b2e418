"""Pins of the benchmark inputs and random-init weights: SHA-256 of the
files synth.py writes for the BASELINE model shapes and of its seeded input
generators, so that a change to either (which would change every number
the bench reports) shows up as a failing test."""
import hashlib
import os

import pytest

import synth

WEIGHTS = {  # (d_model, n_layers, d_state): (bytes, sha256) of seed 0
    (64, 2, 16): (679_172, "a36e2a3558ed92631a89a871000c6afc4bf4b46a94c927da7371e67bac216628"),
    (256, 8, 16): (31_688_708, "888b058eb65d9124eb89e4e8af5aaa9f109486812ff172b62a8d3f86123ab49b"),
}
INPUTS = {
    "gen_c1()": (lambda: synth.gen_c1(), 1_048_576,
                 "93ce11325285c6d12c636b3a61a031ae11e240abbc0dacf3ad5770e12a8dc385"),
    "gen_c2()": (lambda: synth.gen_c2(), 67_108_864,
                 "dbb4f9765b66d949a6d4e19a37d01a5c6258bf84ac723d69ecf1d91665f2541e"),
    "gen_c3(64)": (lambda: synth.gen_c3(64), 262_144,
                   "be153263de9db49cea01420a9fcb4867f2489d6979dbfc13d765d159b5f43016"),
    "gen_c4(1 << 20)": (lambda: synth.gen_c4(1 << 20), 1_048_576,
                        "b84a86b6bafa1b3da3a24160ba96912c26f22976c7891f785197aadf6fdb92a6"),
    "gen_c5(1 << 20)": (lambda: synth.gen_c5(1 << 20), 4_194_304,
                        "0344b1adfebfdfd5d5302dd0a0741c750f8c055b7dbbaa96d8235022ad2c3f55"),
}


@pytest.mark.parametrize("shape", sorted(WEIGHTS))
def test_random_weights_sha256(tmp_path, shape):
    d, L, ds = shape
    p = tmp_path / "w.bin"
    synth.write_random_weights(str(p), d, L, ds, seed=0)
    size, sha = WEIGHTS[shape]
    assert os.path.getsize(p) == size == synth.expected_weight_bytes(d, L, ds)
    assert hashlib.sha256(p.read_bytes()).hexdigest() == sha


@pytest.mark.parametrize("name", sorted(INPUTS))
def test_input_generator_sha256(name):
    fn, size, sha = INPUTS[name]
    b = fn()
    assert len(b) == size
    assert hashlib.sha256(b).hexdigest() == sha
