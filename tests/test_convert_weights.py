"""Weight converter (.pt -> BOA .bin), reference convert_boa_weights.py:153-257.

The expected bytes are assembled here directly from the state dict in the
reference converter's order (convert_boa_weights.py:37-88, 186-239), not
through the converter's own helpers.
"""
import os

import numpy as np
import pytest

import synth

torch = pytest.importorskip("torch")

REF_CKPT = "/root/reference/experiments/cms_experiment/cms_experiment_final_model_fp32_mambav1_64_2_20ep.pt"


def _state_dict(d=64, L=2, ds=16, seed=5, drop_proj_bias=False, ff_net=False):
    sd = {}
    for name, t in synth.random_weight_tensors(d, L, ds, seed=seed):
        if drop_proj_bias and (name.endswith("in_proj.bias") or name.endswith("out_proj.bias")):
            continue
        if ff_net:
            name = name.replace(".ff.", ".ff.net.")
        sd[name] = torch.from_numpy(t.copy())
    return sd


def _expected(sd, fp16):
    """Reference order: embedding; per block ln1, in_proj (w, b or zeros),
    conv1d (w, b if present), x_proj, dt_proj (w, b), A_log, D, out_proj
    (w, b or zeros), ln2, ff.0 (w, b), ff.2 (w, b); head.0 (w, b), head.2 (w, b)."""
    dt = np.float16 if fp16 else np.float32
    parts = [b"BOA\x01" if fp16 else b"BOA\x00"]
    put = lambda a: parts.append(np.asarray(a, np.float32).astype(dt).tobytes())
    put(sd["embedding.weight"].numpy())
    i = 0
    while f"blocks.{i}.ln1.weight" in sd:
        p, m = f"blocks.{i}.", f"blocks.{i}.mamba."
        put(sd[p + "ln1.weight"].numpy())
        put(sd[p + "ln1.bias"].numpy())
        put(sd[m + "in_proj.weight"].numpy())
        put(sd[m + "in_proj.bias"].numpy() if m + "in_proj.bias" in sd
            else np.zeros(sd[m + "in_proj.weight"].shape[0]))
        put(sd[m + "conv1d.weight"].numpy())
        if m + "conv1d.bias" in sd:
            put(sd[m + "conv1d.bias"].numpy())
        for k in ("x_proj.weight", "dt_proj.weight", "dt_proj.bias", "A_log", "D",
                  "out_proj.weight"):
            put(sd[m + k].numpy())
        put(sd[m + "out_proj.bias"].numpy() if m + "out_proj.bias" in sd
            else np.zeros(sd[m + "out_proj.weight"].shape[0]))
        put(sd[p + "ln2.weight"].numpy())
        put(sd[p + "ln2.bias"].numpy())
        ff = p + ("ff.net" if p + "ff.net.0.weight" in sd else "ff")
        for k in (".0.weight", ".0.bias", ".2.weight", ".2.bias"):
            put(sd[ff + k].numpy())
        i += 1
    for k in ("head.0.weight", "head.0.bias", "head.2.weight", "head.2.bias"):
        put(sd[k].numpy())
    return b"".join(parts)


def _run(tmp_path, obj, *extra):
    import convert_weights
    pt = tmp_path / "m.pt"
    out = tmp_path / "m.bin"
    torch.save(obj, pt)
    rc = convert_weights.main(["--model", str(pt), "--output", str(out), *extra])
    return rc, out


@pytest.mark.parametrize("wrap", [None, "state_dict", "model_state_dict"])
def test_fp32_layout(tmp_path, wrap):
    sd = _state_dict()
    rc, out = _run(tmp_path, sd if wrap is None else {wrap: sd, "epoch": 3})
    assert rc == 0
    assert out.read_bytes() == _expected(sd, fp16=False)
    assert out.stat().st_size == synth.expected_weight_bytes(64, 2)


def test_missing_proj_biases_and_ff_net_names(tmp_path):
    sd = _state_dict(drop_proj_bias=True, ff_net=True)
    rc, out = _run(tmp_path, sd)
    assert rc == 0
    assert out.read_bytes() == _expected(sd, fp16=False)


def test_fp16_forced_and_detected(tmp_path):
    sd = _state_dict(d=128, L=1)
    rc, out = _run(tmp_path, sd, "--fp16")
    assert rc == 0 and out.read_bytes() == _expected(sd, fp16=True)
    half = {k: v.half() for k, v in sd.items()}
    rc, out = _run(tmp_path, half)
    assert rc == 0
    blob = out.read_bytes()
    assert blob[:4] == b"BOA\x01" and blob == _expected({k: v.float() for k, v in half.items()}, True)


def test_d_state_32_and_oracle_loads_it(tmp_path, oracle):
    sd = _state_dict(d=64, L=1, ds=32)
    rc, out = _run(tmp_path, sd)
    assert rc == 0
    m = oracle.Model(out, 64, 1, 32)
    data = synth.gen_c1()[:1500]
    assert m.decompress(m.compress(data, chunk_size=500)) == data


def test_other_backbones_rejected(tmp_path):
    sd = {"embedding.weight": torch.zeros(256, 8), "blocks.0.lstm.weight_ih_l0": torch.zeros(4, 4)}
    rc, out = _run(tmp_path, sd)
    assert rc == 1 and not out.exists()


@pytest.mark.skipif(not os.path.exists(REF_CKPT), reason="reference checkpoint not mounted")
def test_reference_checkpoint(tmp_path, oracle):
    import convert_weights
    out = tmp_path / "ckpt.bin"
    info = convert_weights.convert(REF_CKPT, str(out))
    assert (info["d_model"], info["n_layers"], info["d_state"]) == (64, 2, 16)
    assert out.stat().st_size == 679_172
    m = oracle.Model(out, 64, 2)
    zeros = bytes(8192)
    blob = m.compress(zeros, chunk_size=4096)
    assert m.decompress(blob) == zeros and len(blob) * 1.3 < len(zeros)
