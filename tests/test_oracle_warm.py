"""Warm-start mode of the CPU oracle (boa.cpp:310-319, 395-435, 542-559, 608-610).

With warm-start the B = min(gpu_batch, n_chunks) lanes each code S =
ceil(n_chunks / B) chunks in a row, lane b taking chunks b*S + i, and the
model state carries across them.  These tests pin the oracle's warm mode
against facts that do not go through its codec loop:

* the chunk stream of chunk b*S + i equals the range-coder stream built
  from the logits of ONE teacher-forced forward over the concatenation of
  chunks b*S .. b*S + i with a fresh state (so the state that starts a
  chunk has consumed every byte of the lane's earlier chunks);
* with S = 1 (gpu_batch >= n_chunks) the payload equals the cold payload;
* header: flags bit 0 and a 4-byte interleave batch (fp_len = 4);
* decompress inverts compress for ragged tails, truncation and B that does
  not divide the chunk count.
"""
import struct

import numpy as np
import pytest

import synth


def _streams(oracle, blob):
    rc, d = oracle.boa2_parse(blob)
    assert rc == 0
    info = d["info"]
    pay = blob[info.payload_off:]
    return info, d["first"], [np.frombuffer(pay[int(o):int(o) + int(n)], np.uint32)
                              for o, n in zip(d["offsets"], d["lengths"])]


def _expected_warm_stream(oracle, model, data, chunk, nc, B, c):
    S = -(-nc // B)
    b, i = divmod(c, S)
    start = b * S * chunk
    end = min(len(data), (c + 1) * chunk)
    seq = np.frombuffer(data[start:end], np.uint8)
    st = model.new_state(1)
    logits = st.forward_chunk(seq.reshape(1, -1))[0]
    c0 = c * chunk - start               # first position of chunk c in seq
    pos = np.arange(c0, len(seq) - 1)    # predictions for bytes c0+1 .. end-1
    if len(pos) == 0:
        return np.zeros(0, np.uint32)
    cdfs = np.stack([oracle.cdf_quantize(oracle.cdf_build(logits[t])) for t in pos])
    return oracle.encode_cdf_stream(cdfs, seq[pos + 1])


@pytest.mark.parametrize("n,chunk,B", [
    (7 * 96 + 13, 96, 3),   # S = 3, ragged last chunk, lane 2 short by one chunk
    (9 * 64, 64, 4),        # S = 3, B does not divide n_chunks
    (5 * 80, 80, 2),        # S = 3
])
def test_warm_streams_match_concatenated_forward(oracle, w_c1, n, chunk, B):
    data = synth.gen_c1()[:n]
    m = oracle.Model(w_c1, 64, 2)
    blob = m.compress(data, chunk_size=chunk, warm_start=True, gpu_batch=B)
    info, first, streams = _streams(oracle, blob)
    nc = info.n_chunks
    assert nc == -(-n // chunk)
    assert info.flags & 1 and info.interleave_batch == min(B, nc)
    for c in range(nc):
        want = _expected_warm_stream(oracle, m, data, chunk, nc, min(B, nc), c)
        assert np.array_equal(streams[c], want), f"chunk {c}"
        assert first[c] == data[c * chunk]
    assert m.decompress(blob) == data


def test_warm_header_layout(oracle, w_c1):
    data = synth.gen_c1()[:6 * 50 + 7]
    blob = oracle.Model(w_c1, 64, 2).compress(data, chunk_size=50, warm_start=True,
                                              gpu_batch=64)
    assert blob[:4] == b"BOA2"
    flags, = struct.unpack_from("<I", blob, 8)
    assert flags == 1
    assert blob[32] == 4                                   # fp_len
    assert struct.unpack_from("<I", blob, 33)[0] == 7      # min(gpu_batch, 7 chunks)


def test_warm_single_step_equals_cold_payload(oracle, w_c1):
    """S = 1: every lane codes one chunk from zero state, as cold mode does."""
    data = synth.gen_c1()[:5 * 300 + 11]
    m = oracle.Model(w_c1, 64, 2)
    warm = m.compress(data, chunk_size=300, warm_start=True, gpu_batch=64)
    cold = m.compress(data, chunk_size=300)
    iw, _, sw = _streams(oracle, warm)
    ic, _, sc = _streams(oracle, cold)
    assert iw.interleave_batch == 6 and ic.flags == 0
    assert all(np.array_equal(a, b) for a, b in zip(sw, sc))
    assert warm[37:] == cold[33:]                          # payload + index + CRC
    assert m.decompress(warm) == data


def test_warm_state_carry_changes_streams(oracle, w_c1):
    data = synth.gen_c1()[:8 * 200]
    m = oracle.Model(w_c1, 64, 2)
    _, _, sw = _streams(oracle, m.compress(data, chunk_size=200, warm_start=True, gpu_batch=2))
    _, _, sc = _streams(oracle, m.compress(data, chunk_size=200))
    S = 4
    for c in range(8):
        same = np.array_equal(sw[c], sc[c])
        assert same == (c % S == 0), f"chunk {c}: lane starts are cold, the rest carry state"


@pytest.mark.parametrize("n,chunk,B,max_chunks,tile", [
    (0, 64, 4, 0, 0),
    (1, 64, 4, 0, 0),
    (65, 64, 4, 0, 0),           # last chunk of one byte
    (11 * 64 + 5, 64, 3, 0, 16),  # tiled forward
    (20 * 64, 64, 3, 7, 0),       # --max-chunks
    (10 * 1, 1, 3, 0, 0),         # chunk of one byte: the state still consumes it
])
def test_warm_round_trip_edges(oracle, w_c1, n, chunk, B, max_chunks, tile):
    data = synth.gen_c1()[:n]
    m = oracle.Model(w_c1, 64, 2)
    blob = m.compress(data, chunk_size=chunk, warm_start=True, gpu_batch=B,
                      max_chunks=max_chunks, tile=tile)
    keep = n if max_chunks <= 0 else min(n, max_chunks * chunk)
    assert m.decompress(blob) == data[:keep]
    if n:
        untiled = m.compress(data, chunk_size=chunk, warm_start=True, gpu_batch=B,
                             max_chunks=max_chunks)
        assert untiled == blob


def test_warm_bf16_round_trip(oracle, w_c1):
    data = synth.gen_c1()[:9 * 128 + 3]
    m = oracle.Model(w_c1, 64, 2, bf16=True)
    blob = m.compress(data, chunk_size=128, warm_start=True, gpu_batch=4)
    assert m.decompress(blob) == data
