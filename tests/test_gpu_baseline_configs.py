"""GPU parity at the BASELINE configurations' real model depth and lane count.

Every case runs the HIP library through the C ABI on the configuration's
own model (random-init seed 0, as bench.py) and lane count, on short
chunks of the configuration's own input generator so that the CPU oracle
finishes in seconds:

  C1  d64 L2 fp32,            64 lanes, the full 1 MiB input (16 KiB chunks)
  C2  d256 L8 fp32,         1000 lanes x 32 B
  C4  d256 L8 fp32,         4096 lanes x 16 B (Markov source)
  C3  d256 L8 bf16,         8192 lanes x 32 B
  C5  d512 L12 ds32 bf16,  16384 lanes x 16 B

fp32: the containers are byte-identical to the oracle's and round-trip.
bf16: the round trip is byte-exact at the full lane count; the stream bytes
of a chunk subset are within 0.5 % of the oracle's bf16 restatement; logits
of a lane subset are within 2e-2 of the logit scale of the fp32 oracle (the
reference CPU path's precision) and of the bf16 oracle.  Each case also
checks which decode schedule ran (boa_decode_plan): C2 keeps 4 of 8
layers' state in the caches and streams the rest, C4 keeps one (its 160 MiB
of state per layer fills the budget exactly) and runs the unfused-LayerNorm
step above 2048 lanes, C3 and C5 stream every layer.
"""
import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu

TOL_BF16 = 2e-2


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    return torch


def _codec(d, L, ds, lanes, prec="fp32", w=None):
    import boa_hip
    import torch
    c = boa_hip.Codec(d, L, ds, lanes, 0, precision=prec)
    c.set_stream(torch.cuda.current_stream().cuda_stream)
    if w is not None:
        c.load_weights(w)
    return c


def _config_input(name, lanes, chunk):
    """The first `chunk` bytes of each of `lanes` consecutive pieces of the
    configuration's generator output (a prefix of the real input)."""
    n = lanes * chunk
    gen = {"c2": lambda: synth.gen_c2((n + 31) // 32),
           "c3": lambda: synth.gen_c3((n + 4095) // 4096),
           "c4": lambda: synth.gen_c4(n),
           "c5": lambda: synth.gen_c5((n + 3) // 4)}[name]
    return gen()[:n]


def _stream_lengths(oracle, blob):
    rc, info = oracle.boa2_parse(blob)[:2]
    assert rc == 0
    return info


def test_c1_full_input_container(torch_dev, oracle, w_c1):
    """C1 exactly as bench.py runs it: 1 MiB, 64 chunks of 16 KiB, 64 lanes
    (decoded by the persistent d_model-64 kernel)."""
    data = synth.gen_c1()
    assert len(data) == 1 << 20
    c = _codec(64, 2, 16, 64, w=w_c1)
    assert c.decode_plan(64)["persistent"], "C1 decodes in the persistent kernel"
    blob = c.compress(data, chunk_size=16384)
    want = oracle.Model(w_c1, 64, 2).compress(data, chunk_size=16384)
    assert blob == want, f"container differs ({len(blob)} vs {len(want)} bytes)"
    assert c.decompress(blob) == data


@pytest.mark.parametrize("name,lanes,chunk", [("c2", 1000, 32), ("c4", 4096, 16)])
def test_fp32_configs_container_equals_oracle(torch_dev, oracle, make_weights, name, lanes, chunk):
    w = make_weights(256, 8)
    data = _config_input(name, lanes, chunk)
    c = _codec(256, 8, 16, lanes, w=w)
    plan = c.decode_plan(lanes)
    assert not plan["persistent"]
    if name == "c2":
        assert 0 < plan["cached_layers"] < 8, "C2: first layers cached, the rest streamed"
        assert plan["fused_ln"] and plan["fused_xproj"] and not plan["fused_head"]
    else:
        assert plan["cached_layers"] <= 1, "C4: (all but) every layer streamed"
        assert not plan["fused_ln"] and not plan["fused_xproj"] and plan["fused_head"]
    blob = c.compress(data, chunk_size=chunk)
    want = oracle.Model(w, 256, 8).compress(data, chunk_size=chunk)
    assert blob == want, f"{name}: container differs ({len(blob)} vs {len(want)} bytes)"
    assert c.decompress(blob) == data


def test_c2_decode_cache_policies_same_bytes(torch_dev, make_weights):
    """The cached and streamed forms of the decode scan and conv epilogue
    give the same bytes: C2's container decodes with every layer's state
    streamed (budget 0) and with every layer's state cached."""
    w = make_weights(256, 8)
    data = _config_input("c2", 1000, 24)
    c = _codec(256, 8, 16, 1000, w=w)
    blob = c.compress(data, chunk_size=24)
    for budget, want_cached in [(0, 0), (1 << 40, 8), (-1, None)]:
        c.set_state_cache_budget(budget)
        cached = c.decode_plan(1000)["cached_layers"]
        if want_cached is not None:
            assert cached == want_cached
        assert c.decompress(blob) == data, f"budget {budget}"


def _bf16_case(torch, oracle, make_weights, d, L, ds, name, lanes, chunk, subset):
    w = make_weights(d, L, ds)
    data = _config_input(name, lanes, chunk)
    c = _codec(d, L, ds, lanes, prec="bf16", w=w)
    plan = c.decode_plan(lanes)
    assert plan["cached_layers"] == 0 and not plan["persistent"]
    blob = c.compress(data, chunk_size=chunk)
    assert c.decompress(blob) == data, f"{name}: bf16 round trip"
    # stream bytes of the first `subset` chunks against the oracle's bf16
    # restatement (chunks are independent, so the subset's streams are the
    # oracle's compress of those chunks alone)
    got = _stream_lengths(oracle, blob)
    ref = _stream_lengths(oracle, oracle.Model(w, d, L, ds, bf16=True).compress(
        data[:subset * chunk], chunk_size=chunk))
    g = int(sum(got["lengths"][:subset]))
    r = int(sum(ref["lengths"]))
    assert abs(g / r - 1.0) < 5e-3, f"{name}: {g} stream bytes vs oracle {r}"
    c.close()
    # logits of a lane subset: within the bf16 tolerance of the fp32 oracle
    # and of the bf16 oracle
    sub_lanes, T = 16, 24
    tok = np.frombuffer(data[:sub_lanes * T], np.uint8).reshape(sub_lanes, T)
    cs = _codec(d, L, ds, sub_lanes, prec="bf16", w=w)
    cs.reset_state(sub_lanes)
    d_log = torch.zeros(sub_lanes * T * 256, dtype=torch.float32, device="cuda")
    cs.forward_chunk(torch.from_numpy(tok.copy()).cuda(), sub_lanes, T, d_log)
    torch.cuda.synchronize()
    gl = d_log.cpu().numpy().reshape(sub_lanes, T, 256)
    for bf in (False, True):
        want = oracle.Model(w, d, L, ds, bf16=bf).new_state(sub_lanes).forward_chunk(tok)
        scale = np.abs(want).max()
        err = np.abs(gl - want).max()
        assert err <= TOL_BF16 * scale, \
            f"{name}: |gpu bf16 - oracle {'bf16' if bf else 'fp32'}| {err:.3g} > {TOL_BF16} x {scale:.3g}"


def test_c3_bf16_8192_lanes(torch_dev, oracle, make_weights):
    _bf16_case(torch_dev, oracle, make_weights, 256, 8, 16, "c3", 8192, 32, 1024)


def test_c5_bf16_16384_lanes(torch_dev, oracle, make_weights):
    _bf16_case(torch_dev, oracle, make_weights, 512, 12, 32, "c5", 16384, 16, 512)
