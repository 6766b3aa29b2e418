"""The CPU oracle reproduces the frozen fixtures of tests/golden.

The fixtures (written by tests/golden/make_golden.py) are BOA2 containers
of the config-1 model over fixed inputs in cold, warm-start, temperature
and bf16 modes, and a quantised-CDF / coder-stream vector.
"""
import hashlib
import json
import os

import numpy as np
import pytest

import synth

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
MANIFEST = json.load(open(os.path.join(GOLDEN, "manifest.json")))


def fixture(name):
    with open(os.path.join(GOLDEN, name + ".boa"), "rb") as f:
        return f.read()


@pytest.mark.parametrize("name", sorted(MANIFEST["containers"]))
def test_oracle_reproduces_container(oracle, w_c1, name):
    spec = MANIFEST["containers"][name]
    blob = fixture(name)
    assert len(blob) == spec["bytes"]
    assert hashlib.sha256(blob).hexdigest() == spec["sha256"]
    data = synth.gen_c1()[:spec["n"]]
    m = oracle.Model(w_c1, 64, 2, bf16=spec["bf16"])
    assert m.compress(data, chunk_size=spec["chunk"], **spec["options"]) == blob
    assert m.decompress(blob, temperature=spec["options"].get("temperature", 1.0)) == data


def test_oracle_reproduces_cdf_and_coder_vector(oracle):
    v = json.load(open(os.path.join(GOLDEN, "cdf_coder_vector.json")))
    logits = np.array(v["logits"], np.float32)
    q = np.stack([oracle.cdf_quantize(oracle.cdf_build(l)) for l in logits])
    assert np.array_equal(q, np.array(v["qcdf"], np.uint32))
    assert np.all(q[:, 256] == 1 << 24) and np.all(np.diff(q.astype(np.int64), axis=1) >= 1)
    syms = np.array(v["symbols"], np.uint8)
    cdfs = q[np.arange(len(syms)) % 4]
    words = oracle.encode_cdf_stream(cdfs, syms)
    assert words.tolist() == v["words"]
    assert np.array_equal(oracle.decode_cdf_stream(cdfs, len(syms), words), syms)


@pytest.mark.skipif(not __import__("refcpu").host_has_avx512(), reason="host has no AVX-512")
def test_avx512_build_reproduces_the_fixtures(w_c1, weights_dir):
    """The x86-64-v4 (AVX-512) build of the oracle, the timed CPU baseline on
    hosts that have it, writes the same containers as the default build."""
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    names = sorted(MANIFEST["containers"])
    code = (
        "import hashlib, json, sys\n"
        f"sys.path[:0] = [{os.path.join(root, 'oracle')!r}, {os.path.join(root, 'boa-constrictor_amd')!r}]\n"
        "import refcpu, synth\n"
        "assert refcpu.LIB_PATH.endswith('librefcpu_v4.so')\n"
        f"man = json.load(open({os.path.join(GOLDEN, 'manifest.json')!r}))['containers']\n"
        "out = {}\n"
        f"for name in {names!r}:\n"
        "    spec = man[name]\n"
        f"    m = refcpu.Model({str(w_c1)!r}, 64, 2, bf16=spec['bf16'])\n"
        "    blob = m.compress(synth.gen_c1()[:spec['n']], chunk_size=spec['chunk'], **spec['options'])\n"
        "    out[name] = hashlib.sha256(blob).hexdigest()\n"
        "print(json.dumps(out))\n")
    env = dict(os.environ, REFCPU_ISA="v4")
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                       timeout=300, check=True)
    got = json.loads(r.stdout.strip().splitlines()[-1])
    assert got == {n: MANIFEST["containers"][n]["sha256"] for n in names}
