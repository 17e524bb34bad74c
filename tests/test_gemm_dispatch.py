"""Which C entry point each tuner launch reaches (host dispatch only; no GPU).

The harness tuner (harness/cli.py `launch_space`) times the library's own plan and each forced
alternative.  A forced schedule without a split count must run that schedule unsplit, and a
split count must run the split-K entry point with that count; the library's thread-local schedule
setting must hold exactly inside the block.  `_lib.call` is replaced by a recorder, except for the
two host-only planning calls, which run in the real library.
"""

import ctypes

import pytest
import torch

from m5kernels_amd import _lib, hip
from m5kernels_amd.harness import cli

HOST_ONLY = ("m5k_gemm_launch_plan", "m5k_gemm_set_schedule")


def _thread_schedule():
    lib = _lib.load()
    prev = ctypes.c_int(-2)
    assert lib.m5k_gemm_set_schedule(-1, ctypes.byref(prev)) == 0
    assert lib.m5k_gemm_set_schedule(prev.value, None) == 0
    return prev.value


@pytest.fixture
def recorder(monkeypatch):
    calls = []
    real_call = _lib.call

    def call(name, *args):
        if name in HOST_ONLY:
            return real_call(name, *args)
        splits = args[14] if name.startswith("m5k_gemm_i8_splitk") else args[9] if name == "m5k_gemm_f8_splitk" else None
        calls.append((name, splits, _thread_schedule()))

    monkeypatch.setattr(_lib, "call", call)
    monkeypatch.setattr(_lib, "device_tensor", lambda t, name: t.contiguous())
    monkeypatch.setattr(_lib, "stream_of", lambda t: None)
    monkeypatch.setattr(hip, "_cu_count", lambda device: 256)
    hip._i8_schedule.cache_clear()
    hip._f8_splits.cache_clear()
    return calls


@pytest.mark.parametrize("m,n,k", [(128, 7168, 5376), (4096, 5376, 5376)])
def test_each_tuner_launch_reaches_its_entry_point(recorder, m, n, k):
    a = torch.zeros((m, k), dtype=torch.int8)
    b = torch.zeros((n, k), dtype=torch.int8)
    sa, sb = torch.ones(m), torch.ones(n)
    space = cli.launch_space({"m": m, "n": n, "k": k}, "int8")
    assert cli.Launch("plain") in space and cli.Launch("mixed") in space
    for launch in space:
        recorder.clear()
        with launch.active():
            hip.gemm(a, b, "int8", a_scales=sa, b_scales=sb, output_dtype=torch.bfloat16)
        code = -1 if launch.schedule is None else hip.SCHEDULES.index(launch.schedule)
        if launch.splits is not None:
            assert recorder == [("m5k_gemm_i8_splitk", launch.splits, code)], launch
        elif launch.schedule is not None:
            assert recorder == [("m5k_gemm_i8", None, code)], launch
        else:
            planned = hip.splitk_plan(m, n, k, 256)
            if planned > 1:
                assert recorder == [("m5k_gemm_i8_splitk", planned, -1)]
            else:
                assert [c[0] for c in recorder][-1] == "m5k_gemm_i8" and all(c[2] == -1 for c in recorder)
    assert _thread_schedule() == -1  # restored after every block


def test_short_m_plan_splits_but_forced_plain_does_not(recorder):
    # attn_q.m128: the library's plan splits K; the forced "plain" launch must not.
    assert hip.splitk_plan(128, 7168, 5376, 256) > 1
    a = torch.zeros((128, 5376), dtype=torch.int8)
    b = torch.zeros((7168, 5376), dtype=torch.int8)
    with hip.launch_override("plain"):
        hip.gemm(a, b, "int8", a_scales=torch.ones(128), b_scales=torch.ones(7168), output_dtype=torch.bfloat16)
    assert recorder == [("m5k_gemm_i8", None, 0)]


def test_schedule_setting_is_thread_local():
    import threading

    seen = {}
    with hip.launch_override("narrow"):
        t = threading.Thread(target=lambda: seen.setdefault("other", _thread_schedule()))
        t.start()
        t.join()
        seen["this"] = _thread_schedule()
    assert seen == {"other": -1, "this": 2}
    assert _thread_schedule() == -1


def test_set_schedule_rejects_unknown_codes():
    lib = _lib.load()
    assert lib.m5k_gemm_set_schedule(4, None) != 0
    assert lib.m5k_gemm_set_schedule(-2, None) != 0
    assert _thread_schedule() == -1


def test_fp8_short_m_splits_k_and_large_m_or_forced_plain_does_not(recorder):
    # h3 ffn_down at M = 128: 21 tiles of 256 x 256 leave most CUs idle, so the FP8 GEMM splits K
    # over 256 x 128 tiles; at M = 4096, and under a forced schedule, it runs unsplit.
    m, n, k = 128, 5376, 14336
    planned = hip.splitk_plan(m, n, k, 256, skinny=False)
    assert planned > 1 and -(-n // 128) * planned <= 256
    a, b = torch.zeros((m, k), dtype=torch.uint8), torch.zeros((n, k), dtype=torch.uint8)
    kw = dict(a_scales=torch.ones(m), b_scales=torch.ones(n), output_dtype=torch.bfloat16)
    hip.gemm(a, b, "fp8", **kw)
    assert recorder == [("m5k_gemm_f8_splitk", planned, -1)]
    recorder.clear()
    with hip.launch_override("plain"):
        hip.gemm(a, b, "fp8", **kw)
    assert recorder == [("m5k_gemm_f8", None, 0)]
    recorder.clear()
    big = torch.zeros((4096, k), dtype=torch.uint8)
    hip.gemm(big, b, "fp8", a_scales=torch.ones(4096), b_scales=torch.ones(n), output_dtype=torch.bfloat16)
    assert recorder == [("m5k_gemm_f8", None, -1)]


def test_fp8_split_plan_never_needs_the_skinny_tile():
    for m, n, k in [(1, 4096, 4096), (16, 5376, 5376), (128, 7168, 5376), (256, 4096, 16384), (512, 96, 5376)]:
        s8, s = hip.splitk_plan(m, n, k, 256), hip.splitk_plan(m, n, k, 256, skinny=False)
        assert 1 <= s <= 64 and (s == 1 or -(-m // 256) * -(-n // 128) * s <= 256 or -(-m // 256) * -(-n // 256) * s <= 224)
        assert s8 >= 1
