"""The C-ABI library loads on a CPU-only host and exports every entry point
that include/boa_hip.h declares (no compute call is made here)."""
import ctypes

import boa_hip


def test_library_exports_every_declared_symbol():
    lib = boa_hip.lib()
    declared = boa_hip.declared_symbols()
    assert len(declared) > 20
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, f"declared but not exported: {missing}"


def test_host_only_entry_points():
    lib = boa_hip.lib()
    assert lib.boa_weight_file_bytes(256, 8, 16, 0) == 31_688_708
    assert lib.boa_weight_file_bytes(64, 2, 16, 1) == (679_172 - 4) // 2 + 4
    assert lib.boa_num_chunks(67_108_864, 67_109, 0) == 1000
    assert lib.boa_num_chunks(10, 4, 2) == 2
    buf = ctypes.create_string_buffer(b"123456789", 9)
    assert lib.boa_crc32(ctypes.cast(buf, ctypes.c_void_p), 9) == 0xCBF43926
    cfg = boa_hip.Config(256, 8, 16, 1000, 0, 0, 1.0)
    assert lib.boa_estimate_memory(ctypes.byref(cfg), 67_109, 1) > 31_688_708


def test_create_rejects_bad_configs():
    h = ctypes.c_void_p()
    for bad in [boa_hip.Config(513, 8, 16, 10, 0, 0, 1.0),   # d_model above 512 (dt_rank 33)
                boa_hip.Config(0, 8, 16, 10, 0, 0, 1.0),     # d_model
                boa_hip.Config(256, 0, 16, 10, 0, 0, 1.0),   # layers
                boa_hip.Config(256, 8, 24, 10, 0, 0, 1.0),   # d_state
                boa_hip.Config(256, 8, 16, 0, 0, 0, 1.0),    # lanes
                boa_hip.Config(256, 8, 16, 10, 0, 2, 1.0)]:  # precision
        assert boa_hip.lib().boa_create(ctypes.byref(bad), ctypes.byref(h)) == -1
