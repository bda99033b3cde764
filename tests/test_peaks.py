"""The measurement probes of lib/libdih_peaks.so (include/dih_peaks.h): the library exports
what its header declares (CPU), and on the GPU the streaming read really reads every word
(its XOR checksum equals numpy's) and the MFMA loop really runs (its sums are exact)."""
import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "infer.net_amd", "lib", "libdih_peaks.so")
HEADER = os.path.join(ROOT, "include", "dih_peaks.h")


def load():
    lib = ctypes.CDLL(LIB)
    lib.dihp_stream_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    lib.dihp_mfma_loop.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    lib.dihp_mfma_loop_flops.restype = ctypes.c_double
    lib.dihp_mfma_loop_flops.argtypes = [ctypes.c_int, ctypes.c_int]
    lib.dihp_stream_read_pieces.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]
    lib.dihp_stream_read_pieces_blocks.restype = ctypes.c_size_t
    lib.dihp_stream_read_pieces_blocks.argtypes = [ctypes.c_size_t]
    return lib


def test_probe_library_exports_its_header():
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    names = sorted(set(re.findall(r"\b(dihp_[a-z0-9_]+)\s*\(", text)))
    assert len(names) == 6
    lib = load()
    for n in names:
        assert hasattr(lib, n), n
    # 2*32*32*16 flops per MFMA, 4 waves per 256-thread block, 4 chains
    assert lib.dihp_mfma_loop_flops(10, 3) == 3 * 4 * 4 * 10 * 32768.0
    assert lib.dihp_mfma_threads() == 256
    assert lib.dihp_stream_read_pieces_blocks(32768) == 1 and lib.dihp_stream_read_pieces_blocks(32784) == 2


def test_probe_rejects_bad_arguments_before_any_launch():
    lib = load()
    assert lib.dihp_stream_read(None, 16, None, 1, None) != 0
    assert lib.dihp_mfma_loop(None, 1, None, 1, None) != 0


@pytest.mark.gpu
@pytest.mark.parametrize("nbytes,blocks", [(64 << 20, 4096), ((3 << 20) + 48, 333)])
def test_stream_read_checksum(nbytes, blocks):
    import torch
    lib = load()
    rng = np.random.default_rng(nbytes)
    host = rng.integers(0, 1 << 32, size=nbytes // 4, dtype=np.uint32)
    buf = torch.from_numpy(host.view(np.int32)).cuda()
    sink = torch.zeros(blocks, dtype=torch.int32, device="cuda")
    s = torch.cuda.current_stream()
    assert lib.dihp_stream_read(ctypes.c_void_p(buf.data_ptr()), nbytes, ctypes.c_void_p(sink.data_ptr()), blocks,
                                ctypes.c_void_p(s.cuda_stream)) == 0
    torch.cuda.synchronize()
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    assert got == np.bitwise_xor.reduce(host)
    # the one-shot form (a partial last piece when nbytes is not a multiple of 32 KB)
    nb = lib.dihp_stream_read_pieces_blocks(nbytes)
    sink2 = torch.zeros(nb, dtype=torch.int32, device="cuda")
    assert lib.dihp_stream_read_pieces(ctypes.c_void_p(buf.data_ptr()), nbytes, ctypes.c_void_p(sink2.data_ptr()),
                                       ctypes.c_void_p(s.cuda_stream)) == 0
    torch.cuda.synchronize()
    assert np.bitwise_xor.reduce(sink2.cpu().numpy().view(np.uint32)) == np.bitwise_xor.reduce(host)


@pytest.mark.gpu
def test_mfma_loop_sums_are_exact():
    import torch
    lib = load()
    iters, blocks = 64, 8
    ops = torch.full((512,), 0x3F80, dtype=torch.int16, device="cuda")  # bf16 1.0
    out = torch.zeros(blocks * 256, dtype=torch.float32, device="cuda")
    s = torch.cuda.current_stream()
    assert lib.dihp_mfma_loop(ctypes.c_void_p(ops.data_ptr()), iters, ctypes.c_void_p(out.data_ptr()), blocks,
                              ctypes.c_void_p(s.cuda_stream)) == 0
    torch.cuda.synchronize()
    assert bool((out == 1024.0 * iters).all())
    # with every operand 2.0 each product is 4: the sums quadruple
    ops2 = torch.full((512,), 0x4000, dtype=torch.int16, device="cuda")  # bf16 2.0
    assert lib.dihp_mfma_loop(ctypes.c_void_p(ops2.data_ptr()), iters, ctypes.c_void_p(out.data_ptr()), blocks,
                              ctypes.c_void_p(s.cuda_stream)) == 0
    torch.cuda.synchronize()
    assert bool((out == 4096.0 * iters).all())
