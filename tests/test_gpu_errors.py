"""Error paths of the product library (through the C ABI): malformed BOA2
containers and weight files are rejected with BOA_E_FORMAT / BOA_E_IO and a
message, as the reference's reader throws (boa.cpp:195-268) -- never a
crash, a silent zero-filled output or a wrong-size load.  The containers are
built here field by field (header 33 B, payload, IDX2, CRC-32)."""
import struct
import zlib

import pytest

import boa_hip
import synth

pytestmark = pytest.mark.gpu


def _uvarint(x):
    out = bytearray()
    while True:
        b = x & 0x7F
        x >>= 7
        if x:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def boa2(payload, first, lengths, chunk_len, last_len, total=None, version=1, flags=0, fp=b"",
         magic=b"BOA2", crc_xor=0):
    n = len(lengths)
    if total is None:
        total = (n - 1) * chunk_len + last_len if n else 0
    hdr = magic + struct.pack("<IIQIII", version, flags, total, chunk_len, n, last_len)
    hdr += bytes([len(fp)]) + fp
    index = b"IDX2" + bytes(first) + b"".join(_uvarint(v) for v in lengths)
    return hdr + payload + index + struct.pack("<I", zlib.crc32(index) ^ crc_xor)


@pytest.fixture(scope="module")
def codec(w_c1):
    import torch
    assert torch.cuda.is_available(), "GPU tests need a visible MI355X"
    c = boa_hip.Codec(64, 2, 16, 8)
    c.set_stream(torch.cuda.current_stream().cuda_stream)
    c.load_weights(w_c1)
    return c


@pytest.fixture(scope="module")
def good(codec):
    data = synth.gen_c1()[:3 * 500 + 77]
    blob = codec.compress(data, chunk_size=500)
    assert codec.decompress(blob) == data
    return data, blob


def _rc(fn):
    with pytest.raises(boa_hip.BoaError) as ei:
        fn()
    return ei.value.rc, str(ei.value)


def _parts(blob):
    """(payload, first, lengths, chunk_len, last_len) of a cold container."""
    import refcpu
    rc, p = refcpu.boa2_parse(blob)
    assert rc == 0
    info = p["info"]
    payload = blob[info.payload_off: info.idx_off]
    return payload, list(p["first"]), [int(x) for x in p["lengths"]], info.chunk_len, info.last_chunk_len


def test_rebuilt_container_decodes(codec, good):
    data, blob = good
    assert boa2(*_parts(blob)) == blob
    assert codec.decompress(boa2(*_parts(blob))) == data


@pytest.mark.parametrize("case", ["short", "magic", "version", "crc", "no_index", "forged_length",
                                  "chunk_len_zero", "chunk_len_huge", "last_len_zero",
                                  "last_gt_chunk", "total_mismatch", "warm_no_batch",
                                  "warm_batch_gt_chunks"])
def test_malformed_container_rejected(codec, good, case):
    _, blob = good
    payload, first, lens, cl, last = _parts(blob)
    bad = {
        "short": lambda: blob[:20],
        "magic": lambda: b"BOA3" + blob[4:],
        "version": lambda: boa2(payload, first, lens, cl, last, version=2),
        "crc": lambda: boa2(payload, first, lens, cl, last, crc_xor=1),
        "no_index": lambda: blob[:blob.rindex(b"IDX2")],
        "forged_length": lambda: boa2(payload, first, lens[:-1] + [lens[-1] + 1_000_000], cl, last),
        "chunk_len_zero": lambda: boa2(payload, first, lens, 0, last, total=(len(lens) - 1) * cl + last),
        "chunk_len_huge": lambda: boa2(payload, first, lens, (1 << 30) + 1, last),
        "last_len_zero": lambda: boa2(payload, first, lens, cl, 0),
        "last_gt_chunk": lambda: boa2(payload, first, lens, cl, cl + 1),
        "total_mismatch": lambda: boa2(payload, first, lens, cl, last, total=(len(lens) - 1) * cl + last + 1),
        "warm_no_batch": lambda: boa2(payload, first, lens, cl, last, flags=1, fp=struct.pack("<I", 0)),
        "warm_batch_gt_chunks": lambda: boa2(payload, first, lens, cl, last, flags=1,
                                             fp=struct.pack("<I", len(lens) + 1)),
    }[case]()
    rc, msg = _rc(lambda: codec.decompress(bad))
    assert rc == boa_hip.BOA_E_FORMAT, msg
    # the context stays usable after a rejected container
    assert codec.decompress(blob) == good[0]


def test_stream_longer_than_its_chunk_allows(codec):
    """A stream longer than the coder can emit for its chunk length (the
    pitch chunk*10 + 4096 bytes, boa.cpp:338) is rejected before decoding."""
    payload = bytes(5000)
    bad = boa2(payload, [7], [5000], 2, 2)
    rc, msg = _rc(lambda: codec.decompress(bad))
    assert rc == boa_hip.BOA_E_FORMAT and "stream" in msg


def test_weight_file_errors(tmp_path, w_c1):
    import torch
    assert torch.cuda.is_available()
    raw = open(w_c1, "rb").read()
    c = boa_hip.Codec(64, 2, 16, 4)
    trunc = tmp_path / "trunc.bin"
    trunc.write_bytes(raw[:-4])
    rc, msg = _rc(lambda: c.load_weights(trunc))
    assert rc == boa_hip.BOA_E_FORMAT and "expected" in msg
    c3 = boa_hip.Codec(64, 3, 16, 4)  # a 2-layer file for a 3-layer model
    rc, msg = _rc(lambda: c3.load_weights(w_c1))
    assert rc == boa_hip.BOA_E_FORMAT
    rc, msg = _rc(lambda: c.load_weights(tmp_path / "missing.bin"))
    assert rc == boa_hip.BOA_E_IO
    # no weights loaded: the path entry points refuse to run
    rc, msg = _rc(lambda: c.compress(b"abc", chunk_size=2))
    assert rc == boa_hip.BOA_E_STATE
    c.load_weights(w_c1)
    assert c.decompress(c.compress(b"abcdefgh", chunk_size=3)) == b"abcdefgh"
    c.close()
    c3.close()
