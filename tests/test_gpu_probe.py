"""The measurement probes (csrc/probe.hip) behind bench.py's ceiling / stream / launch / mfma
lines: the copy kernel copies exactly (ragged sizes included), the read-only stream kernel reads
buffer lists with ragged and empty buffers without writing anything, and the empty and MFMA
kernels run. These probes are what the hot-path kernels' fractions of the hardware are quoted
against, so they are checked like any other kernel."""
import pytest

pytestmark = pytest.mark.gpu


def _st(dev):
    import torch
    return torch.cuda.current_stream(dev).cuda_stream


@pytest.mark.parametrize("nbytes", [16, 4096 * 16 + 48, (1 << 22) + 16 * 1001])
@pytest.mark.parametrize("U,wg", [(2, 1), (4, 2), (8, 8)])
def test_probe_copy_is_exact(dev, nbytes, U, wg):
    import torch
    from infinitemodel_amd import _lib
    g = torch.Generator(device=dev).manual_seed(nbytes + U)
    src = torch.randint(0, 256, (nbytes + 64,), dtype=torch.uint8, device=dev, generator=g)
    dst = torch.zeros(nbytes + 64, dtype=torch.uint8, device=dev)
    _lib.call("imq_probe_copy", dst.data_ptr(), src.data_ptr(), nbytes, U, wg, _st(dev))
    torch.cuda.synchronize()
    assert torch.equal(dst[:nbytes], src[:nbytes])
    assert not dst[nbytes:].any(), "copy wrote past its end"


@pytest.mark.parametrize("U", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("nt", [0, 1])
def test_probe_stream_reads_ragged_lists_and_writes_nothing(dev, U, nt):
    import torch
    from infinitemodel_amd import _lib
    L = _lib.lib()
    # constant words: every fold is an XOR of an even number of equal words or of zeros, never
    # the kernel's store key, so the sink must stay untouched
    sizes16 = [1, 0, 4096 * U + 3, 7, 0, 65536 + 5]
    bufs = [torch.full((max(n, 1) * 16,), 5, dtype=torch.uint8, device=dev) for n in sizes16]
    ptrs = torch.tensor([b.data_ptr() for b in bufs], dtype=torch.int64, device=dev)
    n16 = torch.tensor(sizes16, dtype=torch.int64, device=dev)
    sink = torch.zeros(int(L.imq_probe_sink_bytes()) // 4, dtype=torch.int32, device=dev)
    for wg in (1, 4, 32):
        _lib.call("imq_probe_stream", ptrs.data_ptr(), n16.data_ptr(), len(bufs), sum(sizes16), U, wg, nt,
                  sink.data_ptr(), sink.numel() * 4, _st(dev))
    torch.cuda.synchronize()
    assert not sink.any()


def test_probe_stream_rejects_bad_arguments(dev):
    import torch
    from infinitemodel_amd import _lib
    L = _lib.lib()
    b = torch.zeros(4096, dtype=torch.uint8, device=dev)
    ptrs = torch.tensor([b.data_ptr()], dtype=torch.int64, device=dev)
    n16 = torch.tensor([256], dtype=torch.int64, device=dev)
    sink = torch.zeros(int(L.imq_probe_sink_bytes()) // 4, dtype=torch.int32, device=dev)
    args = [ptrs.data_ptr(), n16.data_ptr(), 1, 256]
    for u, wg in ((3, 1), (32, 1), (4, 0), (4, 33)):
        assert L.imq_probe_stream(*args, u, wg, 0, sink.data_ptr(), sink.numel() * 4, _st(dev)) == _lib.IMQ_ERR_INVALID
    assert L.imq_probe_stream(*args, 4, 1, 0, sink.data_ptr(), 64, _st(dev)) == _lib.IMQ_ERR_INVALID


def test_probe_empty_and_mfma_run(dev):
    import torch
    from infinitemodel_amd import _lib
    L = _lib.lib()
    sink = torch.zeros(int(L.imq_probe_sink_bytes()) // 4, dtype=torch.int32, device=dev)
    for grid in (1, 256, 4096):
        _lib.call("imq_probe_empty", grid, _st(dev))
    for kind in (0, 1):
        _lib.call("imq_probe_mfma", kind, 64, 2, sink.data_ptr(), sink.numel() * 4, _st(dev))
    torch.cuda.synchronize()
    assert not sink.any()
    assert L.imq_probe_mfma(2, 64, 1, sink.data_ptr(), sink.numel() * 4, _st(dev)) == _lib.IMQ_ERR_INVALID
