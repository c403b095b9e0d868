"""The read probe bench.py times for the per-call floor (wp_read_probe): it
reads what it is given without changing it, and rejects arguments it cannot
take.  Also the program the committed HBM counter summaries are read over
(counter_run)."""
import ctypes

import pytest
import torch

from adapterslotsplusplus_amd import WarpPipeEngine, _lib
from tests.helpers import announce

pytestmark = pytest.mark.gpu


def _probe(engine, buf, nbytes, sink):
    lib = _lib.load()
    return lib.wp_read_probe(engine._handle, ctypes.c_void_p(buf), nbytes, ctypes.c_void_p(sink),
                             ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


def test_read_probe_leaves_its_input():
    engine = WarpPipeEngine()
    buf = torch.arange(1 << 20, dtype=torch.int32, device="cuda")
    sink = torch.zeros(8192, dtype=torch.uint8, device="cuda")
    before = buf.clone()
    for nbytes in (0, 16, 4096, buf.numel() * 4):
        assert _probe(engine, buf.data_ptr(), nbytes, sink.data_ptr()) == _lib.WP_OK
    torch.cuda.synchronize()
    assert torch.equal(buf, before)


def test_read_probe_rejects_bad_arguments():
    engine = WarpPipeEngine()
    buf = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(8192, dtype=torch.uint8, device="cuda")
    assert _probe(engine, buf.data_ptr(), 24, sink.data_ptr()) == _lib.WP_ERR_INVALID      # not a multiple of 16
    assert _probe(engine, buf.data_ptr() + 8, 16, sink.data_ptr()) == _lib.WP_ERR_INVALID  # unaligned
    assert _probe(engine, buf.data_ptr(), -16, sink.data_ptr()) == _lib.WP_ERR_INVALID
    assert _probe(engine, buf.data_ptr(), 16, None) == _lib.WP_ERR_INVALID
    assert "read_probe" in _lib.last_error()


@pytest.mark.parametrize("workload", ["cfg2", "cfg3"])
def test_counter_run_program_runs(workload):
    """The program the committed HBM counter summaries are read over runs to
    its end (one layer, one pass) with a clean error word."""
    from adapterslotsplusplus_amd import counter_run

    announce(f"counter_run --workload {workload}")
    assert counter_run.main(["--workload", workload, "--layers", "1", "--passes", "1"]) == 0
