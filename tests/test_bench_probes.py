"""The measurement probes bench.py loads (libmcq4_bench.so, csrc/bench/mcq4_bench.h).

They are not part of the drop-in library: the CPU tests check that libmcq4.so no
longer exports them and that the bench library's argument checks hold; the GPU
tests check each probe's observable contract."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH_SO = os.path.join(ROOT, "metalops_amd", "_lib", "libmcq4_bench.so")
HEADER = os.path.join(ROOT, "metalops_amd", "csrc", "bench", "mcq4_bench.h")


def _bench():
    import sys
    sys.path.insert(0, ROOT)
    import bench
    return bench.bench_lib()


def test_bench_library_exports_header():
    names = re.findall(r"^int (mcqb_\w+)\(", open(HEADER).read(), re.M)
    assert len(names) == 7
    lib = ctypes.CDLL(BENCH_SO)
    for n in names:
        assert hasattr(lib, n), n


def test_probes_not_in_dropin_library():
    from metalops_amd import _lib
    for n in ("mcq4_read_probe", "mcq4_measure_sclk"):
        assert not hasattr(_lib.lib, n)


def test_probe_argument_checks():
    lib = _bench()
    v = ctypes.c_void_p
    assert lib.mcqb_read_probe(None, 1024, v(256), None) == 1
    assert lib.mcqb_read_probe(v(264), 1024, v(512), None) == 1          # not 16-byte aligned
    assert lib.mcqb_read_probe(v(256), 8, v(512), None) == 1             # fewer than 16 bytes
    assert lib.mcqb_read_tiles(v(256), 4096, 4096, 16, 1, 12, v(512), None) == 1   # waves
    assert lib.mcqb_read_tiles(v(256), 4096, 4096, 24, 1, 16, v(512), None) == 1   # N % tile
    assert lib.mcqb_read_tiles(v(256), 4096, 4096, 16, 129, 16, v(512), None) == 1  # ksplit > K/32
    assert lib.mcqb_read_rows(v(256), 2048, 4096, 96, 1, 8, v(512), None) == 1    # row % piece
    assert lib.mcqb_read_rows(v(256), 2048, 4096, 72, 1, 8, v(512), None) == 1    # piece % 16
    assert lib.mcqb_read_rows(v(256), 2048, 4096, 128, 2049, 8, v(512), None) == 1  # ksplit > rows
    assert lib.mcqb_empty(0, 64, None) == 1
    assert lib.mcqb_empty(1, 2048, None) == 1
    assert lib.mcqb_measure_sclk(None, 10, None) == 1
    assert lib.mcqb_atomic_chain(v(256), 10, 0, v(512), None) == 1
    assert lib.mcqb_exchange(v(256), v(512), 3, 0, 0, 10, None) == 1    # 256 % 6 != 0
    assert lib.mcqb_exchange(v(256), v(512), 8, 3, 0, 10, None) == 1    # store mode


@pytest.mark.gpu
def test_read_probes_leave_sink():
    """Both read probes read and, for data whose workgroup XOR is not the magic
    value, leave the sink untouched."""
    import torch
    lib = _bench()
    src = torch.zeros(18 * 128 * 4096, dtype=torch.uint8, device="cuda")
    sink = torch.full((4,), 7, dtype=torch.int32, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    assert lib.mcqb_read_probe(src.data_ptr(), src.numel() + 5, sink.data_ptr(), s) == 0
    for tc, ks, nw in ((16, 1, 16), (64, 4, 8), (256, 16, 4)):
        assert lib.mcqb_read_tiles(src.data_ptr(), 4096, 4096, tc, ks, nw, sink.data_ptr(), s) == 0
    for pc, ks in ((64, 4), (128, 8)):
        assert lib.mcqb_read_rows(src.data_ptr(), 2048, 4096, pc, ks, 8, sink.data_ptr(), s) == 0
    assert lib.mcqb_empty(256, 256, s) == 0
    torch.cuda.synchronize()
    assert sink.tolist() == [7, 7, 7, 7]


@pytest.mark.gpu
def test_measure_sclk_plausible():
    """Every wave reports shader-clock and 100 MHz real-time ticks; the implied clock
    lies between 300 MHz and 3 GHz (MI355X peaks at 2.4 GHz)."""
    import torch
    lib = _bench()
    ticks = torch.zeros(4096, dtype=torch.int64, device="cuda")
    assert lib.mcqb_measure_sclk(ticks.data_ptr(), 2000, torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    t = ticks.view(-1, 2).double().cpu()
    assert (t[:, 1] > 0).all() and (t[:, 0] > 0).all()
    mhz = 100.0 * t[:, 0] / t[:, 1]
    assert 300.0 < float(mhz.median()) < 3000.0


@pytest.mark.gpu
def test_atomic_chain_counts():
    """Each workgroup's chain adds 1 per iteration to its own two words."""
    import torch
    lib = _bench()
    words = torch.zeros(4 * 64, dtype=torch.int64, device="cuda")
    ticks = torch.zeros(4, dtype=torch.int64, device="cuda")
    assert lib.mcqb_atomic_chain(words.data_ptr(), 50, 4, ticks.data_ptr(), None) == 0
    torch.cuda.synchronize()
    w = words.view(4, 64).cpu()
    assert w[:, :2].sum(dim=1).tolist() == [50, 50, 50, 50]
    assert (ticks.cpu() > 0).all()


@pytest.mark.gpu
def test_exchange_agent_loads_see_stores():
    """An agent-scope atomic load sees another workgroup's agent-scope store on the
    same XCD and on another one (every pair sees its value)."""
    import torch
    lib = _bench()
    slots = torch.zeros(4096, dtype=torch.int64, device="cuda")
    out = torch.zeros(1024, dtype=torch.int64, device="cuda")
    for d in (8, 1):
        slots.zero_()
        assert lib.mcqb_exchange(slots.data_ptr(), out.data_ptr(), d, 1, 1, 200000, None) == 0
        torch.cuda.synchronize()
        h = out.view(256, 4).cpu()
        consumers = [wg for wg in range(256) if (wg // d) % 2 == 1]
        assert all(int(h[wg, 3]) == 1 for wg in consumers)
