"""GPU warm-start parity (boa.cpp:310-319, 395-435, 542-559, 608-610).

The HIP path in warm-start mode writes the oracle's BOA2 bytes (flags bit 0,
4-byte interleave batch, streams in chunk order), decodes its own and the
oracle's containers, and runs more units than lanes in groups of max_lanes.
"""
import os
import subprocess

import pytest

import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    return torch


def _codec(d, L, w, lanes, ds=16, tile=0, precision="fp32"):
    import boa_hip
    import torch
    c = boa_hip.Codec(d, L, ds, lanes, tile, 1.0, precision)
    c.set_stream(torch.cuda.current_stream().cuda_stream)
    c.load_weights(w)
    return c


@pytest.mark.parametrize("n,chunk,lanes,B,max_chunks,tile", [
    (7 * 300 + 13, 300, 8, 3, 0, 0),      # S = 3, ragged last chunk
    (9 * 256, 256, 8, 4, 0, 0),           # B does not divide the chunk count
    (13 * 200 + 1, 200, 2, 5, 0, 0),      # 5 units on 2 lanes: groups of max_lanes
    (20 * 128, 128, 4, 3, 7, 0),          # --max-chunks
    (11 * 512 + 40, 512, 4, 4, 0, 96),    # tiled forward
    (6 * 100, 100, 8, 64, 0, 0),          # B > chunks: S = 1, W = 6
    (0, 64, 4, 4, 0, 0),                  # empty input
    (1, 64, 4, 4, 0, 0),                  # one byte
])
def test_warm_container_matches_oracle(torch_dev, oracle, w_c1, n, chunk, lanes, B,
                                       max_chunks, tile):
    print(f"warm n={n} chunk={chunk} lanes={lanes} B={B} max_chunks={max_chunks} tile={tile}",
          flush=True)
    data = synth.gen_c1()[:n]
    m = oracle.Model(w_c1, 64, 2)
    want = m.compress(data, chunk_size=chunk, warm_start=True, gpu_batch=B,
                      max_chunks=max_chunks, tile=tile)
    c = _codec(64, 2, w_c1, lanes, tile=tile)
    c.set_warm_start(B)
    got = c.compress(data, chunk_size=chunk, max_chunks=max_chunks)
    assert got == want, f"container differs ({len(got)} vs {len(want)} bytes)"
    keep = n if max_chunks <= 0 else min(n, max_chunks * chunk)
    assert c.decompress(got) == data[:keep]
    c.set_warm_start(0)          # the decoder takes the batch from the header
    assert c.decompress(got) == data[:keep]
    assert m.decompress(got) == data[:keep]


def test_warm_c2_shape_decoder_lanes_differ(torch_dev, oracle, make_weights):
    """d256 x 2 layers; the decoder runs fewer lanes than the interleave batch."""
    w = make_weights(256, 2)
    data = synth.gen_c2(4096)[:10 * 600 + 77]
    want = oracle.Model(w, 256, 2).compress(data, chunk_size=600, warm_start=True, gpu_batch=4)
    enc = _codec(256, 2, w, 4)
    enc.set_warm_start(4)
    got = enc.compress(data, chunk_size=600)
    assert got == want
    dec = _codec(256, 2, w, 3)
    assert dec.decompress(got) == data


def test_warm_bf16_round_trip(torch_dev, make_weights):
    """bf16: GPU compress and decode agree bit for bit, so the round trip holds."""
    w = make_weights(128, 1)
    data = synth.gen_c3(8)[:9 * 400 + 5]
    c = _codec(128, 1, w, 4, precision="bf16")
    c.set_warm_start(3)
    blob = c.compress(data, chunk_size=400)
    assert c.decompress(blob) == data


def test_warm_lane_starts_are_cold_streams(torch_dev, oracle, w_c1):
    """A unit's first chunk starts from zero state, so its stream is the cold
    stream of that chunk; later chunks of the unit carry state and differ."""
    data = synth.gen_c1()[:12 * 256]
    c = _codec(64, 2, w_c1, 8)
    cold = c.compress(data, chunk_size=256)
    c.set_warm_start(3)                      # S = 4: units start at chunks 0, 4, 8
    warm = c.compress(data, chunk_size=256)
    assert c.decompress(warm) == data

    def streams(blob):
        rc, d = oracle.boa2_parse(blob)
        assert rc == 0
        pay = blob[d["info"].payload_off:]
        return [pay[int(o):int(o) + int(n)] for o, n in zip(d["offsets"], d["lengths"])]

    for k, (w, cs) in enumerate(zip(streams(warm), streams(cold))):
        assert (w == cs) == (k % 4 == 0), f"chunk {k}"


def test_cli_warm_start_matches_oracle(torch_dev, oracle, w_c1, tmp_path):
    exe = os.path.join(os.path.dirname(__file__), "..", "boa-constrictor_amd", "boa")
    data = synth.gen_c1()[:12 * 1000 + 17]
    src = tmp_path / "in.bin"
    src.write_bytes(data)
    boa_f = tmp_path / "out.boa"
    back = tmp_path / "back.bin"
    subprocess.run([exe, "compress", str(w_c1), str(src), str(boa_f), "64", "2",
                    "--gpu-batch", "5", "--chunk-size", "1000", "--warm-start"], check=True,
                   timeout=120)
    want = oracle.Model(w_c1, 64, 2).compress(data, chunk_size=1000, warm_start=True,
                                              gpu_batch=5)
    assert boa_f.read_bytes() == want
    subprocess.run([exe, "decompress", str(w_c1), str(boa_f), str(back), "64", "2",
                    "--gpu-batch", "2"], check=True, timeout=120)
    assert back.read_bytes() == data
