"""The prefill dispatch rule (worker_quant.py:1235-1335 and the forward's fall-through,
817-853) on the CPU, against hand-worked expectations of the reference's decision procedure:

* ``_prefill_bench_m``: the row bucket of INFINITEMODEL_PREFILL_CHUNK (default 2048; a value
  <= 1 or unparsable keeps 2048).
* ``_naive_threshold`` (the measured decision as a pure rule over timings): naive must beat the
  fused time at the chunk bucket by the 13% margin (strictly), else 0 = fused at every M; when
  it does, each halved bucket down to 16 keeps naive while it still beats the fused time
  extrapolated linearly in rows, and the first bucket where it does not ends the descent (smaller
  buckets are never timed).
* ``_bench_large_m_naive``: one measurement per (tag, N, K_pad, group) key, cached; a failing
  measurement returns 0 and is not cached; the IM_LARGE_M_NAIVE=0 switch.
* the forward: a call whose row bucket reaches ``_naive_m_min`` skips the fused op and runs the
  naive ``F.linear(x, _dequant(x.dtype))``; smaller buckets keep the fused op; threshold 0 keeps
  the fused op everywhere."""
import pytest
import torch
import torch.nn.functional as F

from infinitemodel_amd import worker_quant as wq
from tests import _cases as C


class _Timings:
    """naive_ms(m) from a table, recording which row counts were timed."""

    def __init__(self, table):
        self.table = table
        self.calls = []

    def __call__(self, m):
        self.calls.append(m)
        return self.table[m]


@pytest.mark.parametrize("raw,bucket", [(None, 2048), ("", 2048), ("2048", 2048), ("1500", 2048), ("300", 512),
                                        ("16", 16), ("17", 32), ("1", 2048), ("0", 2048), ("abc", 2048)])
def test_prefill_bench_m_is_the_chunk_bucket(monkeypatch, raw, bucket):
    if raw is None:
        monkeypatch.delenv("INFINITEMODEL_PREFILL_CHUNK", raising=False)
    else:
        monkeypatch.setenv("INFINITEMODEL_PREFILL_CHUNK", raw)
    assert wq._prefill_bench_m() == bucket


def test_m_bucket_is_next_power_of_two():
    assert [wq._m_bucket(m) for m in (0, 1, 2, 3, 16, 17, 33, 64, 65, 1500, 2048)] == \
        [0, 1, 2, 4, 16, 32, 64, 64, 128, 2048, 2048]


def test_naive_never_wins_keeps_fused_everywhere():
    # fused 10 ms at 2048 rows; naive 9 ms is a 10% win, short of the 13% margin
    t = _Timings({2048: 9.0})
    assert wq._naive_threshold(2048, 10.0, t) == 0
    assert t.calls == [2048]


@pytest.mark.parametrize("naive,expect", [(8.71, 0), (8.69, 2048)])
def test_margin_is_strict_thirteen_percent(naive, expect):
    # 0.87 * 10 ms = 8.7 ms: naive must be below it
    t = _Timings({2048: naive, 1024: 1e9})
    assert wq._naive_threshold(2048, 10.0, t) == expect


def test_naive_wins_only_at_the_chunk_bucket():
    # fused per row = 10 / 2048 ms; at 1024 rows naive must be < 0.87 * 5 = 4.35 ms: 5 ms is not
    t = _Timings({2048: 5.0, 1024: 5.0})
    assert wq._naive_threshold(2048, 10.0, t) == 2048
    assert t.calls == [2048, 1024]


def test_naive_wins_down_to_sixteen_rows():
    # naive at half the extrapolated fused time at every bucket: the descent runs to 16 and stops
    # there (8 rows are never timed)
    per_row = 10.0 / 2048
    table = {m: 0.5 * per_row * m for m in (2048, 1024, 512, 256, 128, 64, 32, 16, 8)}
    t = _Timings(table)
    assert wq._naive_threshold(2048, 10.0, t) == 16
    assert t.calls == [2048, 1024, 512, 256, 128, 64, 32, 16]


def test_descent_stops_at_the_first_losing_bucket():
    # wins at 2048 and 1024 (1 ms < 0.87 * 5 = 4.35), loses at 512 (100 ms), would win at 256: the
    # threshold is 1024 and 256 is never timed
    t = _Timings({2048: 1.0, 1024: 1.0, 512: 100.0, 256: 0.001})
    assert wq._naive_threshold(2048, 10.0, t) == 1024
    assert t.calls == [2048, 1024, 512]


def test_extrapolation_is_linear_in_rows():
    # fused 8 ms at 2048 -> 2 ms extrapolated at 512 rows; the bound there is 0.87 * 2 = 1.74 ms
    per = {2048: 1.0, 1024: 1.0, 512: 1.73, 256: 0.9}
    assert wq._naive_threshold(2048, 8.0, _Timings(per)) == 512
    per[512] = 1.75
    assert wq._naive_threshold(2048, 8.0, _Timings(per)) == 1024


@pytest.mark.parametrize("top,calls,expect", [(16, [16], 16), (32, [32, 16], 16), (512, [512, 256], 512)])
def test_small_chunk_buckets(top, calls, expect):
    per_row = 10.0 / top
    table = {m: 0.5 * per_row * m for m in (512, 32, 16)}
    table[256] = 1e9
    t = _Timings(table)
    assert wq._naive_threshold(top, 10.0, t) == expect
    assert t.calls == calls


# ---- _bench_large_m_naive: keying, caching, failure and the off switch ------------------------------
class _FakeMod:
    """What _bench_large_m_naive reads from a bound module: _fused, in_features, group_size,
    _dequant."""

    def __init__(self, N, in_f, in_pad, G=128, op=None):
        self.qweight = torch.zeros(N, in_pad // 2, dtype=torch.uint8)
        self._fused = (self.qweight, ("s", "z"), op or (lambda x, qw, g, pair: None), in_pad)
        self.in_features = in_f
        self.group_size = G
        self._w = torch.zeros(N, in_f, dtype=torch.bfloat16)

    def _dequant(self, dtype):
        return self._w.to(dtype)


def _scripted_device_ms(monkeypatch, seq):
    """Replace the device timer: each call runs fn once and returns the next scripted time."""
    it = iter(seq)
    calls = []

    def fake(fn, dev, iters, warmup):
        fn()
        calls.append(1)
        return next(it)

    monkeypatch.setattr(wq, "_device_ms", fake)
    return calls


def test_bench_is_keyed_and_cached(monkeypatch):
    monkeypatch.setenv("INFINITEMODEL_PREFILL_CHUNK", "64")
    monkeypatch.setattr(wq, "_LARGE_M_NAIVE", True)
    monkeypatch.setattr(wq, "_LARGE_M_CHOICE", {})
    # fused 10 ms at 64 rows; naive 1 ms at 64 and 32 (wins: < 0.87 * 5), 100 ms at 16 -> 32
    calls = _scripted_device_ms(monkeypatch, [10.0, 1.0, 1.0, 100.0])
    m = _FakeMod(48, 96, 128)
    assert wq._bench_large_m_naive(m, "int4") == 32
    assert len(calls) == 4
    assert wq._LARGE_M_CHOICE == {("int4", 48, 128, 128): 32}
    # same key: cached, no timing; another N or tag: measured again
    assert wq._bench_large_m_naive(_FakeMod(48, 96, 128), "int4") == 32
    assert len(calls) == 4
    _scripted_device_ms(monkeypatch, [10.0, 9.0])
    assert wq._bench_large_m_naive(_FakeMod(40, 96, 128), "int4") == 0
    assert wq._LARGE_M_CHOICE[("int4", 40, 128, 128)] == 0


def test_bench_failure_returns_zero_uncached(monkeypatch):
    monkeypatch.setattr(wq, "_LARGE_M_NAIVE", True)
    monkeypatch.setattr(wq, "_LARGE_M_CHOICE", {})

    def boom(fn, dev, iters, warmup):
        raise RuntimeError("timer failed")

    monkeypatch.setattr(wq, "_device_ms", boom)
    assert wq._bench_large_m_naive(_FakeMod(48, 96, 128), "int4") == 0
    assert wq._LARGE_M_CHOICE == {}


def test_bench_off_switch(monkeypatch):
    monkeypatch.setattr(wq, "_LARGE_M_NAIVE", False)
    monkeypatch.setattr(wq, "_LARGE_M_CHOICE", {})
    monkeypatch.setattr(wq, "_device_ms", lambda *a, **k: pytest.fail("timed with the switch off"))
    assert wq._bench_large_m_naive(_FakeMod(48, 96, 128), "int4") == 0


# ---- the forward's fall-through ---------------------------------------------------------------------
def _bound_mod(op):
    N, K, G = 48, 300, 128
    c = C.int4_case(N, K, G, 3)
    m = wq._quant4_linear_cls()(C.u8(c["q"], "cpu"), C.to_torch(c["s"], "bf16", "cpu"),
                                C.to_torch(c["z"], "bf16", "cpu"), None, K, G)
    m._fused = (m.qweight, (m.scale, m.zero), op, 384)
    m._fused_tried = True
    return m


def test_forward_falls_through_from_the_threshold_bucket():
    seen = []

    def op(x, qw, g, pair):
        seen.append(x.shape[0])
        return torch.zeros(x.shape[0], qw.shape[0], dtype=torch.bfloat16)

    m = _bound_mod(op)
    m._naive_m_min = 64
    for rows, fused in ((1, True), (16, True), (32, True), (33, False), (64, False), (100, False)):
        seen.clear()
        x = torch.randn(rows, 300).to(torch.bfloat16)
        y = m(x)
        if fused:
            assert seen == [rows] and not y.any()
        else:
            assert seen == []
            assert torch.equal(y, F.linear(x, m._dequant(torch.bfloat16)) if rows < 16 else
                               F.linear(x.float(), m._dequant(torch.float32)).to(torch.bfloat16))
    # leading dims count as rows: 2 x 20 = 40 rows -> bucket 64 -> naive
    seen.clear()
    m(torch.randn(2, 20, 300).to(torch.bfloat16))
    assert seen == []


def test_threshold_zero_or_no_qweight_keeps_fused():
    seen = []

    def op(x, qw, g, pair):
        seen.append(x.shape[0])
        return torch.zeros(x.shape[0], 48, dtype=torch.bfloat16)

    m = _bound_mod(op)
    m._naive_m_min = 0
    m(torch.randn(4096, 300).to(torch.bfloat16))
    assert seen == [4096]
    m._naive_m_min = 64
    m.qweight = None          # the reference keeps the fused op when qweight was released
    m(torch.randn(128, 300).to(torch.bfloat16))
    assert seen == [4096, 128]
