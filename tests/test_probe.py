"""bench.py's HBM read-rate probe (crane_amd/csrc/probe/hbm_probe.hip): a
measurement helper built beside the library, not part of its C ABI.  The
probe's rate means something only if it reads every byte once: the xor of
its per-workgroup words must be the xor of the whole buffer."""
import ctypes
import os

import numpy as np
import pytest

PROBE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "crane_amd", "libcrane_probe.so")


def _probe():
    if not os.path.exists(PROBE):
        pytest.fail("libcrane_probe.so is not built: run __graft_entry__.build()")
    lib = ctypes.CDLL(PROBE)
    lib.crane_probe_read.restype = ctypes.c_int
    lib.crane_probe_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    lib.crane_probe_workgroups.restype = ctypes.c_int64
    lib.crane_probe_workgroups.argtypes = [ctypes.c_int64, ctypes.c_int]
    return lib


def test_probe_rejects_bad_arguments():
    """Checked on the host before any launch (no GPU needed)."""
    lib = _probe()
    buf = ctypes.create_string_buffer(64)
    addr = (ctypes.addressof(buf) + 15) // 16 * 16
    assert lib.crane_probe_read(None, 16, addr, 8, None) == -1
    assert lib.crane_probe_read(addr, 16, None, 8, None) == -1
    assert lib.crane_probe_read(addr, 24, addr, 8, None) == -1          # not a multiple of 16
    assert lib.crane_probe_read(addr, 0, addr, 8, None) == -1
    assert lib.crane_probe_read(addr, 1 << 31, addr, 8, None) == -1     # past the 32-bit offsets
    assert lib.crane_probe_read(addr, 16, addr, 12, None) == -1         # 8, 16 or 32 loads
    assert lib.crane_probe_read(addr + 4, 16, addr, 8, None) == -1      # unaligned
    assert lib.crane_probe_workgroups(1, 8) == 1
    assert lib.crane_probe_workgroups(32768, 8) == 1 and lib.crane_probe_workgroups(32784, 8) == 2
    assert lib.crane_probe_workgroups(320 * 1000 * 1000, 32) == 2442


@pytest.mark.gpu
@pytest.mark.parametrize("nbytes,loads", [(16, 8), (4096, 16), (1 << 20, 32), (48 * (1 << 20) + 48, 8),
                                          (320 * 1000 * 1000, 32)])
def test_probe_reads_every_chunk(gpu, nbytes, loads):
    import torch
    lib = _probe()
    print(f"probe {nbytes} B, {loads} loads a thread", flush=True)
    rng = np.random.default_rng(nbytes + loads)
    words = rng.integers(0, 2 ** 32, size=nbytes // 4, dtype=np.uint64).astype(np.uint32)
    src = torch.from_numpy(words.view(np.int32)).to(gpu)
    sink = torch.zeros(int(lib.crane_probe_workgroups(nbytes, loads)), dtype=torch.int32, device=gpu)
    st = torch.cuda.current_stream(gpu).cuda_stream
    assert lib.crane_probe_read(src.data_ptr(), nbytes, sink.data_ptr(), loads, st) == 0
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    assert got == np.bitwise_xor.reduce(words)
