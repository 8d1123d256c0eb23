"""The read-bandwidth probe (libsparsebench_probe.so, sbp_read), which the
roofline ceilings of bench_baselines.py come from: its argument checks on the
CPU (no kernel runs), and both read modes on the GPU.

On the GPU each lane folds what it read into one word (XOR) and stores it to
sink only when it equals `key`: over zeros every fold is 0, so key 0 must
leave sink[0..256) all zero and key 1 must leave it untouched.
"""

import ctypes

import pytest
import torch

from sparsebench_amd import _lib

MODES = {"vector": 0, "lds_dma": 1}


@pytest.fixture(scope="module")
def probe():
    path = _lib.LIB_PATH.with_name("libsparsebench_probe.so")
    if not path.exists():
        from sparsebench_amd.build import build

        build()
    _lib.lib()  # torch's HIP runtime first, then the tool library
    handle = ctypes.CDLL(str(path))
    handle.sbp_read.restype = ctypes.c_int
    handle.sbp_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_uint32, ctypes.c_void_p,
                                ctypes.c_void_p]
    handle.sbp_last_error.restype = ctypes.c_char_p
    return handle


def test_read_probe_rejects(probe) -> None:
    buf = ctypes.create_string_buffer(4096)
    p = ctypes.addressof(buf) + (-ctypes.addressof(buf)) % 16
    sink = p + 1024
    cases = [
        ((None, 1 << 20, 0, 1, sink, None), "null buffer"),
        ((p, 1 << 20, 0, 1, None, None), "null buffer"),
        ((p + 4, 1 << 20, 0, 1, sink, None), "16-byte aligned"),
        ((p, 17, 0, 1, sink, None), "positive multiple of 16"),
        ((p, 0, 0, 1, sink, None), "positive multiple of 16"),
        ((p, 1000, 1, 1, sink, None), "whole MiB"),
        ((p, 1 << 20, 7, 1, sink, None), "mode must be"),
    ]
    for args, msg in cases:
        assert probe.sbp_read(*args) == 1, msg
        assert msg in probe.sbp_last_error().decode()


@pytest.mark.gpu
@pytest.mark.parametrize("mode", list(MODES))
def test_read_probe_reads(probe, mode: str) -> None:
    data = torch.zeros(4 << 20, dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    for key, want in ((1, 0xFFFFFFFF), (0, 0)):
        sink = torch.full((256,), -1, dtype=torch.int32, device="cuda")
        rc = probe.sbp_read(data.data_ptr(), data.numel(), MODES[mode], key, sink.data_ptr(), stream)
        assert rc == 0, probe.sbp_last_error().decode()
        torch.cuda.synchronize()
        assert (sink.cpu().numpy().astype("uint32") == want).all(), (mode, key)
