"""The group-synchronous decode step (fp32, d_model 256, up to 1024 lanes).

One launch runs a whole decode step: its phases are the launch chain's
kernels (LayerNorm + in_proj + conv, x_proj + scan, out_proj, LayerNorm +
FF1, FF2, head.1, head.2 + CDF + search + coder), and the 16 workgroups of
each 64-lane group meet at a barrier of their own between phases.

Each case compresses with the GPU, requires the container to equal the
CPU oracle's byte for byte, and decodes it twice: with the group step and
with the launch chain (boa_set_decode_group(0)), both back to the input.
Lane counts cover one lane, partial 16-lane tiles and 64-lane groups, all
16 groups (1024 lanes) and the C2 model at its 1000 lanes; ragged last
chunks, several batches per call, both cache policies of the state and
warm-start are covered too.
"""
import pytest

import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    return torch


def _codec(L, lanes, w):
    import boa_hip
    import torch
    c = boa_hip.Codec(256, L, 16, lanes, 0)
    c.set_stream(torch.cuda.current_stream().cuda_stream)
    c.load_weights(w)
    c.set_decode_group(True)
    return c


def _data(n):
    return synth.gen_c2((n + 31) // 32)[:n]


@pytest.mark.parametrize("lanes,chunk,L,cut", [
    (1, 40, 2, 0),       # one lane: one group, one 16-lane tile
    (17, 64, 2, 9),      # a partial second tile, ragged last chunk
    (100, 48, 2, 5),     # a partial second group
    (512, 24, 2, 0),     # 8 groups: one per XCD
    (1024, 16, 2, 3),    # all 16 groups
    (1000, 20, 8, 7),    # the C2 model at its lane count
])
def test_group_step_matches_oracle_and_chain(torch_dev, oracle, make_weights, lanes, chunk, L, cut):
    w = make_weights(256, L)
    data = _data(lanes * chunk - cut)
    c = _codec(L, lanes, w)
    assert c.decode_plan(lanes)["group_step"], "this shape decodes with the group step"
    blob = c.compress(data, chunk_size=chunk)
    want = oracle.Model(w, 256, L).compress(data, chunk_size=chunk)
    assert blob == want, f"container differs ({len(blob)} vs {len(want)} bytes)"
    assert c.decompress(blob) == data, "group step round trip"
    c.set_decode_group(False)
    assert not c.decode_plan(lanes)["group_step"]
    assert c.decompress(blob) == data, "launch-chain round trip"
    c.set_decode_group(True)
    assert c.decompress(blob) == data, "group step again after the chain"
    c.close()


def test_group_step_several_batches(torch_dev, oracle, make_weights):
    """150 chunks through 64 lanes: three batches (64, 64, 22 lanes), the
    groups' decoded positions restarting for each."""
    w = make_weights(256, 2)
    data = _data(150 * 30 - 11)
    c = _codec(2, 64, w)
    blob = c.compress(data, chunk_size=30)
    assert blob == oracle.Model(w, 256, 2).compress(data, chunk_size=30)
    assert c.decode_plan(64)["group_step"] and c.decode_plan(22)["group_step"]
    assert c.decompress(blob) == data
    c.close()


@pytest.mark.parametrize("budget,cached", [(0, 0), (1 << 40, 3)])
def test_group_step_state_cache_policies(torch_dev, make_weights, budget, cached):
    """Every layer's state streamed past the caches, or every layer cached."""
    w = make_weights(256, 3)
    data = _data(300 * 24)
    c = _codec(3, 300, w)
    blob = c.compress(data, chunk_size=24)
    c.set_state_cache_budget(budget)
    plan = c.decode_plan(300)
    assert plan["group_step"] and plan["cached_layers"] == cached
    assert c.decompress(blob) == data
    c.close()


def test_group_step_warm_start(torch_dev, oracle, make_weights):
    """Warm-start: units of 3 consecutive chunks over 40 lanes; the carry
    step between a unit's chunks runs the launch chain, the batch steps the
    group step."""
    w = make_weights(256, 2)
    data = _data(120 * 32 - 5)
    c = _codec(2, 40, w)
    c.set_warm_start(40)
    blob = c.compress(data, chunk_size=32)
    ref = oracle.Model(w, 256, 2)
    assert blob == ref.compress(data, chunk_size=32, warm_start=True, gpu_batch=40)
    assert c.decompress(blob) == data
    c.close()
