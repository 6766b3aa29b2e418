"""GPU parity across model shapes, weight formats, options and edge cases.

Each case runs the HIP library through the C ABI and the CPU oracle on the
same seeded inputs, and requires identical logit bits, identical BOA2 bytes
and byte-identical round trips.  Shapes cover the BASELINE configs' models
at reduced depth (C2 d256, C5 d512 with d_state 32) so the oracle finishes
in seconds.
"""
import os
import subprocess

import numpy as np
import pytest

import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    return torch


def _codec(d, L, ds=16, lanes=64, tile=0, w=None, temperature=1.0):
    import boa_hip
    import torch
    c = boa_hip.Codec(d, L, ds, lanes, tile, temperature)
    c.set_stream(torch.cuda.current_stream().cuda_stream)
    if w is not None:
        c.load_weights(w)
    return c


@pytest.mark.parametrize("d,L,ds", [(80, 2, 16), (128, 1, 16), (256, 2, 16), (512, 1, 32)])
def test_forward_and_step_bit_exact(torch_dev, oracle, make_weights, d, L, ds):
    """Chunk-mode logits equal the oracle's; step-mode logits equal chunk mode."""
    torch = torch_dev
    w = make_weights(d, L, ds)
    lanes, T = 5, 24
    rng = np.random.default_rng(d + L + ds)
    tok = rng.integers(0, 256, size=(lanes, T), dtype=np.uint8)
    want = oracle.Model(w, d, L, ds).new_state(lanes).forward_chunk(tok)
    c = _codec(d, L, ds, lanes=lanes, w=w)
    c.reset_state(lanes)
    d_log = torch.zeros(lanes * T * 256, dtype=torch.float32, device="cuda")
    c.forward_chunk(torch.from_numpy(tok).cuda(), lanes, T, d_log)
    torch.cuda.synchronize()
    got = d_log.cpu().numpy().reshape(lanes, T, 256)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        f"d={d} L={L} ds={ds}: max |diff| {np.abs(got - want).max()}"
    c.reset_state(lanes)
    d_s = torch.zeros(lanes * 256, dtype=torch.float32, device="cuda")
    for t in range(T):
        c.step_batch(torch.from_numpy(np.ascontiguousarray(tok[:, t])).cuda(), lanes, d_s, True)
        st = d_s.cpu().numpy().reshape(lanes, 256)
        assert np.array_equal(st.view(np.uint32), want[:, t].view(np.uint32)), f"step {t}"


@pytest.mark.parametrize("d,L,ds", [(128, 1, 16), (256, 1, 16), (512, 1, 32)])
def test_fp32_many_lanes_step_equals_chunk_and_round_trip(torch_dev, make_weights, d, L, ds):
    """From 2048 lanes on, the fp32 decode step's GEMMs run their many-lane
    tile forms (32 x 32 and 64-lane wave tiles, a partial last tile at 2100
    lanes): step logits stay bit-identical to chunk logits, and a container
    of 2101 chunks (one decode batch) round-trips byte for byte."""
    torch = torch_dev
    w = make_weights(d, L, ds)
    lanes, T = 2100, 5
    rng = np.random.default_rng(11 + d)
    tok = rng.integers(0, 256, size=(lanes, T), dtype=np.uint8)
    c = _codec(d, L, ds, lanes=2200, w=w)
    c.reset_state(lanes)
    d_log = torch.zeros(lanes * T * 256, dtype=torch.float32, device="cuda")
    c.forward_chunk(torch.from_numpy(tok).cuda(), lanes, T, d_log)
    torch.cuda.synchronize()
    got = d_log.cpu().numpy().reshape(lanes, T, 256)
    c.reset_state(lanes)
    d_s = torch.zeros(lanes * 256, dtype=torch.float32, device="cuda")
    for t in range(T):
        c.step_batch(torch.from_numpy(np.ascontiguousarray(tok[:, t])).cuda(), lanes, d_s, True)
        st = d_s.cpu().numpy().reshape(lanes, 256)
        assert np.array_equal(st.view(np.uint32), got[:, t].view(np.uint32)), f"step {t}"
    data = synth.gen_c2(2700)[:2100 * 40 + 7]
    blob = c.compress(data, chunk_size=40)
    assert c.decompress(blob) == data


@pytest.mark.parametrize("d,ds,prec", [(64, 16, "fp32"), (80, 16, "fp32"), (256, 16, "fp32"),
                                       (64, 16, "bf16"), (256, 16, "bf16"), (512, 32, "bf16")])
def test_scan_forms_agree(torch_dev, oracle, make_weights, d, ds, prec):
    """The compress scan runs token-blocked (16 threads per channel, passes
    of 32 tokens at d_state 16 and 16 at d_state 32) on small grids (under
    one wave per SIMD) and one thread per channel with scalar-loaded delta
    rows otherwise: the same lanes' logits are bit-identical between a small
    and a large batch, and (fp32) equal to the oracle's.  70 tokens give
    whole passes, a ragged last pass and a ragged 16-token block."""
    import boa_hip
    torch = torch_dev
    w = make_weights(d, 1, ds)
    di = 2 * d
    big = -(-64 * 1024 // di)  # the first lane count on the scalar-load form
    small, T = 6, 70
    rng = np.random.default_rng(7 + d + ds)
    tok = rng.integers(0, 256, size=(big, T), dtype=np.uint8)
    out = []
    for lanes in (small, big):
        c = boa_hip.Codec(d, 1, ds, lanes, 0, precision=prec)
        c.set_stream(torch.cuda.current_stream().cuda_stream)
        c.load_weights(w)
        c.reset_state(lanes)
        d_log = torch.zeros(lanes * T * 256, dtype=torch.float32, device="cuda")
        c.forward_chunk(torch.from_numpy(np.ascontiguousarray(tok[:lanes])).cuda(), lanes, T, d_log)
        torch.cuda.synchronize()
        out.append(d_log.cpu().numpy().reshape(lanes, T, 256)[:small])
        c.close()
    assert np.array_equal(out[0].view(np.uint32), out[1].view(np.uint32))
    if prec == "fp32":
        want = oracle.Model(w, d, 1, ds).new_state(small).forward_chunk(tok[:small])
        assert np.array_equal(out[1].view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("lanes", [6, 1000, 1500, 5000])
def test_persistent_decode_lanes_per_block(torch_dev, oracle, make_weights, lanes):
    """The d_model-64 persistent decode gives each block 4, 8 or 16 lanes,
    the fewest whose grid fits the CUs (on 256 CUs: 4 up to 1024 lanes, 8 up
    to 2048, then 16), and leaves the MFMA rows beyond them inert.  Every
    block size, with a partial last block and a ragged last chunk, gives the
    oracle's container bytes and a byte-identical round trip."""
    w = make_weights(64, 2, 16)
    chunk = 24
    rng = np.random.default_rng(lanes)
    data = rng.integers(0, 256, size=lanes * chunk - 5, dtype=np.uint8).tobytes()
    c = _codec(64, 2, 16, lanes=lanes, w=w)
    assert c.decode_plan(lanes)["persistent"]
    blob = c.compress(data, chunk_size=chunk)
    want = oracle.Model(w, 64, 2).compress(data, chunk_size=chunk)
    assert blob == want, f"container differs ({len(blob)} vs {len(want)} bytes)"
    assert c.decompress(blob) == data
    c.close()


def test_layernorm_in_gemm_epilogues(torch_dev, oracle, make_weights):
    """At d_model 256 with 16384 rows or more in a call (128 x 256 GEMM
    tiles) the fp32 pass runs LN2 in out_proj's epilogue and the next layer's
    LN1 in FF2's.  Its logits equal, bit for bit, those of the same tokens in
    short calls (separate LayerNorm kernels), and the oracle's for two lanes."""
    import boa_hip
    torch = torch_dev
    d, L, ds = 256, 2, 16
    w = make_weights(d, L, ds)
    lanes, T, Ts = 66, 256, 32  # 16896 rows in one call, 2112 in each short one
    rng = np.random.default_rng(23)
    tok = rng.integers(0, 256, size=(lanes, T), dtype=np.uint8)
    c = boa_hip.Codec(d, L, ds, lanes, 0, precision="fp32")
    c.set_stream(torch.cuda.current_stream().cuda_stream)
    c.load_weights(w)

    def chunk(t0, t1):
        out = torch.zeros(lanes * (t1 - t0) * 256, dtype=torch.float32, device="cuda")
        c.forward_chunk(torch.from_numpy(np.ascontiguousarray(tok[:, t0:t1])).cuda(), lanes,
                        t1 - t0, out)
        torch.cuda.synchronize()
        return out.cpu().numpy().reshape(lanes, t1 - t0, 256)

    c.reset_state(lanes)
    whole = chunk(0, T)
    c.reset_state(lanes)
    parts = np.concatenate([chunk(t, t + Ts) for t in range(0, T, Ts)], axis=1)
    c.close()
    assert np.array_equal(whole.view(np.uint32), parts.view(np.uint32))
    pick = [0, lanes - 1]
    want = oracle.Model(w, d, L, ds).new_state(2).forward_chunk(np.ascontiguousarray(tok[pick]))
    assert np.array_equal(whole[pick].view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("d,ds,prec", [(256, 16, "fp32"), (256, 16, "bf16"), (512, 32, "bf16")])
def test_state_carries_across_modes(torch_dev, make_weights, d, ds, prec):
    """The recurrent state moves between the chunk layout (forward_chunk) and
    the step layout (step_batch; bf16 keeps its conv state as bf16 there):
    chunk then steps, and steps then chunk, give the logits of one chunk pass
    over all tokens, bit for bit."""
    import boa_hip
    torch = torch_dev
    w = make_weights(d, 2, ds)
    lanes, T1, T2 = 7, 9, 6
    T = T1 + T2
    rng = np.random.default_rng(11 + d + ds)
    tok = rng.integers(0, 256, size=(lanes, T), dtype=np.uint8)
    c = boa_hip.Codec(d, 2, ds, lanes, 0, precision=prec)
    c.set_stream(torch.cuda.current_stream().cuda_stream)
    c.load_weights(w)

    def chunk(t0, t1):
        out = torch.zeros(lanes * (t1 - t0) * 256, dtype=torch.float32, device="cuda")
        c.forward_chunk(torch.from_numpy(np.ascontiguousarray(tok[:, t0:t1])).cuda(), lanes,
                        t1 - t0, out)
        torch.cuda.synchronize()
        return out.cpu().numpy().reshape(lanes, t1 - t0, 256)

    def steps(t0, t1):
        out = []
        d_s = torch.zeros(lanes * 256, dtype=torch.float32, device="cuda")
        for t in range(t0, t1):
            c.step_batch(torch.from_numpy(np.ascontiguousarray(tok[:, t])).cuda(), lanes, d_s, True)
            torch.cuda.synchronize()
            out.append(d_s.cpu().numpy().reshape(lanes, 256).copy())
        return np.stack(out, axis=1)

    c.reset_state(lanes)
    want = chunk(0, T)
    c.reset_state(lanes)
    got = np.concatenate([chunk(0, T1), steps(T1, T)], axis=1)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), "chunk -> steps"
    c.reset_state(lanes)
    got = np.concatenate([steps(0, T1), chunk(T1, T)], axis=1)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), "steps -> chunk"


def _same_container(oracle, w, d, L, ds, data, chunk, lanes, tile=0, temperature=1.0,
                    max_chunks=0):
    m = oracle.Model(w, d, L, ds)
    want = m.compress(data, chunk_size=chunk, tile=tile, max_chunks=max_chunks,
                      temperature=temperature)
    c = _codec(d, L, ds, lanes=lanes, tile=tile, w=w, temperature=temperature)
    got = c.compress(data, chunk_size=chunk, max_chunks=max_chunks)
    assert got == want, f"container differs ({len(got)} vs {len(want)} bytes)"
    n = len(data) if max_chunks <= 0 else min(len(data), max_chunks * chunk)
    assert c.decompress(got) == data[:n]
    assert m.decompress(got, temperature=temperature) == data[:n]
    return got


def test_container_c2_shape(torch_dev, oracle, make_weights):
    data = synth.gen_c2(4096)[:9 * 700 + 3]
    _same_container(oracle, make_weights(256, 2), 256, 2, 16, data, 700, lanes=4)


def test_container_c5_shape_d_state_32(torch_dev, oracle, make_weights):
    data = synth.gen_c5(2048)[:5 * 512 + 77]
    _same_container(oracle, make_weights(512, 1, 32), 512, 1, 32, data, 512, lanes=6)


def test_container_d_model_80(torch_dev, oracle, make_weights):
    """d_model 80 (dt_rank 5), the shape of the reference's
    ..._mambav1_80_1_20.pt, with two layers and ragged chunks."""
    data = synth.gen_c1()[:7 * 600 + 41]
    _same_container(oracle, make_weights(80, 2), 80, 2, 16, data, 600, lanes=5)


def test_container_markov_source(torch_dev, oracle, w_c1):
    data = synth.gen_c4(8 * 1500)
    _same_container(oracle, w_c1, 64, 2, 16, data, 1500, lanes=8)


def test_container_fp16_weights(torch_dev, oracle, make_weights):
    w16 = make_weights(64, 2, 16, seed=3, fp16=True)
    data = synth.gen_c1()[:6 * 900]
    _same_container(oracle, w16, 64, 2, 16, data, 900, lanes=6)


def test_container_temperature(torch_dev, oracle, w_c1):
    data = synth.gen_c1()[:5 * 800 + 5]
    blob = _same_container(oracle, w_c1, 64, 2, 16, data, 800, lanes=8, temperature=0.7)
    assert blob != oracle.Model(w_c1, 64, 2).compress(data, chunk_size=800)


@pytest.mark.parametrize("n,chunk,lanes,max_chunks", [
    (0, 512, 4, 0),          # empty input: header, empty index
    (1, 512, 4, 0),          # one byte: one chunk, no coded symbols
    (513, 512, 4, 0),        # last chunk of one byte
    (7 * 300, 300, 3, 0),    # three batches of lanes
    (10 * 256, 256, 4, 4),   # --max-chunks truncation
    (37 * 333 - 100, 333, 37, 0),  # three 16-lane decode blocks, the last one partial
    (45 * 200 + 5, 200, 20, 0),    # batches of 20 lanes, a last batch of 6, a 5-byte chunk
])
def test_container_edges(torch_dev, oracle, w_c1, n, chunk, lanes, max_chunks):
    data = synth.gen_c1()[:n]
    _same_container(oracle, w_c1, 64, 2, 16, data, chunk, lanes=lanes, max_chunks=max_chunks)


def test_container_tiles_shorter_than_the_conv(torch_dev, oracle, w_c1):
    """Tiles of 100 tokens over 403-byte chunks end with a 2-token tile: the
    conv reads its inputs and writes its state across tile boundaries,
    including tiles shorter than its 4 taps."""
    data = synth.gen_c1()[:6 * 403]
    _same_container(oracle, w_c1, 64, 2, 16, data, 403, lanes=3, tile=100)


def test_container_4096_lanes(torch_dev, oracle, w_c1):
    """C4's lane count (4096 chunks decoded in one batch) at a short chunk."""
    data = synth.gen_c4(4096 * 40 + 17)
    _same_container(oracle, w_c1, 64, 2, 16, data, 40, lanes=4096)


def test_cli_round_trip_matches_oracle(torch_dev, oracle, w_c1, tmp_path):
    """The C++ CLI (boa.cpp's command line) writes the oracle's container."""
    exe = os.path.join(os.path.dirname(__file__), "..", "boa-constrictor_amd", "boa")
    data = synth.gen_c1()[:12 * 1000 + 17]
    src = tmp_path / "in.bin"
    src.write_bytes(data)
    boa_f = tmp_path / "out.boa"
    back = tmp_path / "back.bin"
    subprocess.run([exe, "compress", str(w_c1), str(src), str(boa_f), "64", "2",
                    "--gpu-batch", "5", "--chunk-size", "1000"], check=True, timeout=120)
    want = oracle.Model(w_c1, 64, 2).compress(data, chunk_size=1000)
    assert boa_f.read_bytes() == want
    subprocess.run([exe, "decompress", str(w_c1), str(boa_f), str(back), "64", "2",
                    "--gpu-batch", "5"], check=True, timeout=120)
    assert back.read_bytes() == data
