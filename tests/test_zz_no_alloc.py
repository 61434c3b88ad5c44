"""imq_linear_w4_noalloc (static per-device scratch, no allocation) against imq_linear_w4 with a
caller workspace, through the C ABI. Both run the same kernels with the same split plans, so the
outputs must be bit-identical; each pair is two calls in a row with the second one smaller, so
the scratch holds the first call's partials when the second runs."""
import pytest

from infinitemodel_amd import _lib

pytestmark = pytest.mark.gpu


def _case(dev, M, N, K, seed):
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    ng = K // 128
    q = torch.randint(0, 256, (N, K // 2), dtype=torch.uint8, device=dev, generator=g)
    s = (torch.rand((N, ng), device=dev, generator=g) * 0.004 + 0.001).to(torch.bfloat16)
    z = torch.randint(0, 16, (N, ng), device=dev, generator=g).to(torch.bfloat16)
    x = torch.randn((M, K), device=dev, generator=g).to(torch.bfloat16)
    return x, q, s, z


def _args(x, q, s, z, y):
    M, K = x.shape
    N = q.shape[0]
    return [x.data_ptr(), x.stride(0), M, K, q.data_ptr(), q.stride(0), s.data_ptr(), s.stride(0), s.stride(1),
            _lib.IMQ_DT_BF16, z.data_ptr(), z.stride(0), z.stride(1), _lib.IMQ_DT_BF16, N, 128, y.data_ptr(),
            y.stride(0)]


def _run_pair(dev, M, N, K, seed):
    import torch
    L = _lib.lib()
    x, q, s, z = _case(dev, M, N, K, seed)
    st = torch.cuda.current_stream(dev).cuda_stream
    need = int(L.imq_linear_w4_workspace_bytes(M, K, N, 128, q.stride(0), x.stride(0), s.stride(0), s.stride(1),
                                                _lib.IMQ_DT_BF16, z.stride(0), z.stride(1), _lib.IMQ_DT_BF16))
    assert need <= L.imq_linear_workspace_bytes(M, N, K)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    y_ref = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    y_na = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
    rc = L.imq_linear_w4(*_args(x, q, s, z, y_ref), ws.data_ptr(), ws.numel(), st)
    assert rc == 0, L.imq_strerror(rc)
    rc = L.imq_linear_w4_noalloc(*_args(x, q, s, z, y_na), st)
    assert rc == 0, L.imq_strerror(rc)
    torch.cuda.synchronize(dev)
    assert torch.equal(y_ref.view(torch.int16), y_na.view(torch.int16)), (M, N, K)
    assert torch.isfinite(y_ref.float()).all()
    return need


@pytest.mark.parametrize("first,second", [
    # prefill split-K: C4 14336 -> 4096 at M=512 (32 MiB of partials), then a smaller split-K shape
    ((512, 4096, 14336), (64, 4096, 4096)),
    # decode K-split: C2 down at M=16 (3.7 MB of partials), then down at M=8
    ((16, 4096, 14336), (8, 4096, 14336)),
])
def test_noalloc_matches_workspace_entry(dev, first, second):
    n1 = _run_pair(dev, *first, seed=11)
    n2 = _run_pair(dev, *second, seed=12)
    assert 0 < n2 < n1 <= _lib.IMQ_NOALLOC_SCRATCH_BYTES


def test_noalloc_decode_rows_without_partials(dev):
    """M <= 4 takes the line kernel and C2 gate_up at M = 16 the wave-split kernel (no partials
    either): still identical, twice in a row, and the allocation-free entry takes wave-split shapes
    of any width (no scratch needed)."""
    assert _run_pair(dev, 4, 6144, 4096, seed=13) == 0
    assert _run_pair(dev, 1, 4096, 4096, seed=14) == 0
    assert _run_pair(dev, 16, 28672, 4096, seed=16) == 0
    assert _run_pair(dev, 16, 1 << 19, 4096, seed=17) == 0


def test_noalloc_rejects_oversize_on_gpu(dev):
    """A shape whose partials exceed the scratch is refused with IMQ_ERR_SCRATCH and launches
    nothing (the output keeps its contents)."""
    import torch
    L = _lib.lib()
    M, N, K = 16, 1 << 19, 14336     # K-split: 14 splits x 16 x 524288 x 4 B = 448 MiB of partials
    x, q, s, z = _case(dev, M, N, K, seed=15)
    need = L.imq_linear_w4_workspace_bytes(M, K, N, 128, q.stride(0), x.stride(0), s.stride(0), s.stride(1),
                                           _lib.IMQ_DT_BF16, z.stride(0), z.stride(1), _lib.IMQ_DT_BF16)
    assert need == 14 * M * N * 4 > _lib.IMQ_NOALLOC_SCRATCH_BYTES
    y = torch.zeros((M, N), dtype=torch.bfloat16, device=dev)
    rc = L.imq_linear_w4_noalloc(*_args(x, q, s, z, y), torch.cuda.current_stream(dev).cuda_stream)
    assert rc == _lib.IMQ_ERR_SCRATCH
    torch.cuda.synchronize(dev)
    assert not y.any()
