"""Host-side op contracts (CPU): the same exception type for the same condition as the
reference's Python ops, raised before any device work, and no silent CPU path."""

from __future__ import annotations

import pytest
import torch

from m5kernels_amd import gemm, quantize, rotate, rotate_quantize


def test_quantize_rejections():
    with pytest.raises(ValueError):
        quantize(torch.zeros(8), "int8")  # not [rows, K]
    with pytest.raises(ValueError, match="unknown"):
        quantize(torch.zeros(2, 8), "int4")
    with pytest.raises(ValueError, match="MXINT8 requires K divisible by 32"):
        quantize(torch.zeros(2, 40), "mxint8")
    with pytest.raises(ValueError, match="ROCm device"):  # mxint8 is computed, on the GPU only
        quantize(torch.zeros(2, 64), "mxint8")
    with pytest.raises(ValueError, match="float16, bfloat16 or float32"):
        quantize(torch.zeros(2, 8, dtype=torch.int8), "int8")


def test_cpu_tensors_are_refused_not_computed():
    with pytest.raises(ValueError, match="ROCm device"):
        quantize(torch.ones(2, 8), "int8")
    with pytest.raises(ValueError, match="ROCm device"):
        gemm(torch.ones(2, 8, dtype=torch.bfloat16), torch.ones(3, 8, dtype=torch.bfloat16), "bf16")


def _i8(m, k):
    return torch.zeros(m, k, dtype=torch.int8)


def test_gemm_shape_and_mode_rejections():
    with pytest.raises(ValueError, match="K mismatch"):
        gemm(_i8(2, 8), _i8(3, 9), "int8")
    with pytest.raises(NotImplementedError, match="stride"):  # reference test_metal.py:137-143
        gemm(torch.zeros(2, 96, dtype=torch.uint8), torch.zeros(3, 96, dtype=torch.uint8), "fp8")
    with pytest.raises(NotImplementedError, match="overflow"):
        gemm(_i8(1, 133145), _i8(1, 133145), "int8")
    with pytest.raises(ValueError, match="scales required"):
        gemm(_i8(2, 8), _i8(3, 8), "int8")
    with pytest.raises(KeyError):
        gemm(_i8(2, 8), _i8(3, 8), "int4")
    with pytest.raises(ValueError, match="divisible by 32"):
        gemm(torch.zeros(2, 8, dtype=torch.int8), torch.zeros(3, 8, dtype=torch.int8), "mxint8",
             a_scales=torch.zeros(2, 1, dtype=torch.uint8), b_scales=torch.zeros(3, 1, dtype=torch.uint8))
    with pytest.raises(ValueError, match="scales required"):
        gemm(torch.zeros(2, 32, dtype=torch.int8), torch.zeros(3, 32, dtype=torch.int8), "mxint8")
    with pytest.raises(ValueError, match="uint8 exponents"):
        gemm(torch.zeros(2, 32, dtype=torch.int8), torch.zeros(3, 32, dtype=torch.int8), "mxint8",
             a_scales=torch.zeros(2, dtype=torch.float32), b_scales=torch.zeros(3, 1, dtype=torch.uint8))
    with pytest.raises(ValueError):
        gemm(_i8(2, 8), _i8(3, 8), "int8", tile=(64, 64))


def test_gemm_epilogue_rejections():
    sa, sb = torch.ones(2), torch.ones(3)
    kw = dict(a_scales=sa, b_scales=sb)
    res = torch.zeros(2, 3, dtype=torch.bfloat16)
    gate = torch.zeros(3, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="both residual and gate"):
        gemm(_i8(2, 8), _i8(3, 8), "int8", residual=res, output_dtype=torch.bfloat16, **kw)
    with pytest.raises(NotImplementedError, match="INT8 and BF16"):
        gemm(torch.zeros(2, 128, dtype=torch.uint8), torch.zeros(3, 128, dtype=torch.uint8), "fp8",
             residual=res, gate=gate, **kw)
    with pytest.raises(NotImplementedError, match="explicit BF16"):
        gemm(_i8(2, 8), _i8(3, 8), "int8", residual=res, gate=gate, **kw)
    with pytest.raises(NotImplementedError, match="combining"):
        gemm(_i8(2, 8), _i8(3, 8), "int8", residual=res, gate=gate, bias=torch.zeros(3),
             output_dtype=torch.bfloat16, **kw)
    with pytest.raises(ValueError, match="residual must"):
        gemm(_i8(2, 8), _i8(3, 8), "int8", residual=res.float(), gate=gate, output_dtype=torch.bfloat16, **kw)
    with pytest.raises(ValueError, match="gate must have shape"):
        gemm(_i8(2, 8), _i8(3, 8), "int8", residual=res, gate=gate[:2], output_dtype=torch.bfloat16, **kw)
    with pytest.raises(ValueError, match="gate_row_map"):
        gemm(_i8(2, 8), _i8(3, 8), "int8", residual=res, gate=torch.zeros(4, 3, dtype=torch.bfloat16),
             gate_row_map=torch.zeros(2, dtype=torch.int64), output_dtype=torch.bfloat16, **kw)
    with pytest.raises(ValueError, match="bias_row_map requires"):
        gemm(_i8(2, 8), _i8(3, 8), "int8", bias_row_map=torch.zeros(2, dtype=torch.int32), **kw)
    with pytest.raises(NotImplementedError, match="INT8 only"):
        gemm(torch.zeros(2, 8, dtype=torch.bfloat16), torch.zeros(3, 8, dtype=torch.bfloat16), "bf16",
             bias=torch.zeros(3))
    with pytest.raises(ValueError, match="float32"):
        gemm(_i8(2, 8), _i8(3, 8), "int8", bias=torch.zeros(3, dtype=torch.float16), **kw)
    with pytest.raises(ValueError, match="shape \\[N\\]"):
        gemm(_i8(2, 8), _i8(3, 8), "int8", bias=torch.zeros(4), **kw)
    with pytest.raises(ValueError, match="mapped bias"):
        gemm(_i8(2, 8), _i8(3, 8), "int8", bias=torch.zeros(4, 2), bias_row_map=torch.zeros(2, dtype=torch.int32),
             **kw)


@pytest.mark.parametrize("fn", [rotate, rotate_quantize])
def test_hadamard_rejections(fn):
    x = torch.zeros(3, 768)
    signs = torch.ones(768, dtype=torch.int8)
    for block, error, message in [
        (33, ValueError, "power of two"),
        (2.0, ValueError, "power of two"),
        (True, ValueError, "power of two"),
        (2048, NotImplementedError, "supported block sizes"),
        (16, NotImplementedError, "supported block sizes"),
        (512, NotImplementedError, "divisible"),
    ]:
        with pytest.raises(error, match=message):
            fn(x, block, signs)
    with pytest.raises(ValueError, match="signs"):
        fn(x, 256, torch.ones(768))
    with pytest.raises(ValueError, match="signs"):
        fn(x, 256, torch.ones(767, dtype=torch.int8))
    with pytest.raises(ValueError, match="shape"):
        fn(torch.zeros(0, 768), 256, signs)
    with pytest.raises(ValueError, match="dtype"):
        fn(torch.zeros(3, 768, dtype=torch.int32), 256, signs)


def test_rotate_implementation_switch():
    x, signs = torch.zeros(3, 256), torch.ones(256, dtype=torch.int8)
    with pytest.raises(NotImplementedError):
        rotate(x, 256, signs, implementation="mlx")
    with pytest.raises(ValueError, match="unknown Hadamard implementation"):
        rotate(x, 256, signs, implementation="cuda")


def test_rms_quantize_validation():
    """rms_quant.py:56-100: metadata errors, checked before any device work."""
    from m5kernels_amd import rms_quantize

    x, g, s = torch.zeros(2, 64), torch.ones(64), torch.ones(64, dtype=torch.int8)
    with pytest.raises(ValueError, match="shape"):
        rms_quantize(torch.zeros(64), g, s)
    with pytest.raises(ValueError, match="gamma"):
        rms_quantize(x, torch.ones(64, dtype=torch.float16), s)
    with pytest.raises(ValueError, match="signs"):
        rms_quantize(x, g, torch.ones(64))
    with pytest.raises(ValueError, match="power of two"):
        rms_quantize(x, g, s, 3)
    with pytest.raises(NotImplementedError, match="supported blocks"):
        rms_quantize(x, g, s, 16)
    with pytest.raises(NotImplementedError, match="divisible"):
        rms_quantize(torch.zeros(2, 96), torch.ones(96), torch.ones(96, dtype=torch.int8), 64)
    with pytest.raises(NotImplementedError, match="threadgroup"):
        rms_quantize(x, g, s, threads=64)
    with pytest.raises(ValueError, match="boolean"):
        rms_quantize(x, g, s, fold_scale=1)
    with pytest.raises(ValueError, match="epsilon"):
        rms_quantize(x, g, s, epsilon=0)
    with pytest.raises(ValueError, match="identifier"):
        rms_quantize(x, g, s, tag="1bad")
    with pytest.raises(ValueError, match="ROCm device"):
        rms_quantize(x, g, s)


def test_grouped_qkv_validation():
    from m5kernels_amd import projection_qkv_rope

    g = torch.ones(128, dtype=torch.bfloat16)
    cs = torch.ones(4, 48, dtype=torch.bfloat16)
    a = torch.zeros(4, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="heads\\*3\\*128"):
        projection_qkv_rope(a, torch.zeros(256, 64, dtype=torch.bfloat16), g, g, cs, cs, "bf16")
    with pytest.raises(NotImplementedError):
        projection_qkv_rope(a, torch.zeros(384, 64, dtype=torch.bfloat16), g, g, cs, cs, "fp8")
    with pytest.raises(ValueError, match="k_gamma"):
        projection_qkv_rope(a, torch.zeros(384, 64, dtype=torch.bfloat16), g, torch.ones(64, dtype=torch.bfloat16),
                            cs, cs, "bf16")
    with pytest.raises(ValueError, match="ROCm device"):
        projection_qkv_rope(a, torch.zeros(384, 64, dtype=torch.bfloat16), g, g, cs, cs, "bf16")


def test_shift_split_validation():
    """norm_hadamard_gemm.py:39-44: the split policy needs RMS, round_output=fp32, one_read and a
    known bias backend; the tables need matching shapes.  All raised before device work."""
    from m5kernels_amd import norm_shift_split_gemm, shift_split_condition

    x, s = torch.zeros(2, 256, dtype=torch.bfloat16), torch.ones(256, dtype=torch.int8)
    wq, ws, c, b = torch.zeros(3, 256, dtype=torch.int8), torch.ones(3), torch.ones(256), torch.zeros(3)
    with pytest.raises(NotImplementedError, match="round_output=fp32"):
        norm_shift_split_gemm(x, wq, ws, s, c, b, round_output="input")
    with pytest.raises(NotImplementedError, match="round_output=fp32"):
        norm_shift_split_gemm(x, wq, ws, s, c, b, norm="layer")
    with pytest.raises(NotImplementedError, match="passes=one_read"):
        norm_shift_split_gemm(x, wq, ws, s, c, b, passes="two_read")
    with pytest.raises(ValueError, match="ROCm device"):
        norm_shift_split_gemm(x, wq, ws, s, c, b)
    g = torch.ones(256, dtype=torch.bfloat16)
    w = torch.zeros(3, 256, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError, match="bias preparation backend"):
        shift_split_condition(g, g, g, w, bias_backend="numpy")
    with pytest.raises(ValueError, match="\\[K\\] or \\[P,K\\]"):
        shift_split_condition(g, g, torch.ones(2, 256, dtype=torch.bfloat16), w)
    with pytest.raises(ValueError, match="gamma must have shape"):
        shift_split_condition(torch.ones(255, dtype=torch.bfloat16), g, g, w)
    with pytest.raises(ValueError, match="bfloat16 shift"):
        shift_split_condition(g, g, g.float(), w, bias_backend="mpp-bf16-to-fp32")
    with pytest.raises(ValueError, match="ROCm device"):
        shift_split_condition(g, g, g, w)


def test_launch_plan_decisions(monkeypatch):
    """The library's GEMM schedule on 256 CUs (host query, no GPU).  Whole rounds keep the plain
    launch.  A partial last round keeps the leading whole rounds as 256 x 256 tiles and halves
    the rest when one shorter round saves 5% or more.  256 x 224 tiles (16 x 16 modes) take
    shapes whose narrow tile count fills whole rounds.  Every choice here measured faster on
    MI355X than the plain launch (mixed 6-22%, narrow 3-6%), bit-identically."""
    from m5kernels_amd.hip import launch_plan

    expected = {
        (4096, 4096): ("plain", -1),     # 256 tiles: one whole round
        (9914, 14336): ("plain", -1),    # 2184 tiles: 8.5 rounds
        (9914, 4096): ("mixed", 512),    # 624 tiles: 2 rounds + 224 halves
        (4096, 5376): ("mixed", 256),    # 336 tiles: 1 round + 160 halves
        (4096, 14336): ("mixed", 768),   # 896 tiles: 3 rounds + 256 halves
        (2048, 4096): ("mixed", 0),      # 128 tiles: all halved
        (300, 200): ("mixed", 0),
        (4096, 7168): ("narrow", -1),    # 448 tiles = 1.75 rounds; 512 narrow tiles = 2 rounds
        (1024, 14336): ("narrow", -1),   # 224 tiles; 256 narrow tiles
        (2048, 5120): ("narrow", -1),    # ragged last narrow tile column (5120 = 22 x 224 + 192)
    }
    for (m, n), plan in expected.items():
        assert launch_plan("int8", m, n, 256) == plan, (m, n)
        assert launch_plan("bf16", m, n, 256) == plan, (m, n)
    # FP8 and FP32 use 32 x 32 blocks and have no narrow grid.
    assert launch_plan("fp8", 4096, 7168, 256) == ("plain", -1)
    assert launch_plan("fp32", 9914, 4096, 256) == ("mixed", 512)
    for m in range(1, 12000, 331):
        for n in (96, 1536, 4096, 5376, 7168):
            sched, full = launch_plan("int8", m, n, 256)
            tiles = -(-m // 256) * -(-n // 256)
            if sched == "mixed":
                assert full % 256 == 0 and 0 <= full < tiles and tiles % 256
            else:
                assert full == -1
    monkeypatch.setenv("M5K_GEMM_MIXED_TILES", "0")
    assert launch_plan("int8", 9914, 4096, 256) == ("narrow", -1)  # 741 narrow tiles: 3 rounds
    assert launch_plan("fp32", 9914, 4096, 256) == ("plain", -1)
    monkeypatch.setenv("M5K_GEMM_NARROW_TILES", "0")
    assert launch_plan("int8", 9914, 4096, 256) == ("plain", -1)
    assert launch_plan("int8", 4096, 7168, 256) == ("plain", -1)
    monkeypatch.delenv("M5K_GEMM_MIXED_TILES")
    monkeypatch.delenv("M5K_GEMM_NARROW_TILES")
    with pytest.raises(RuntimeError, match="cus must be positive"):
        launch_plan("int8", 9914, 4096, 0)


def test_forced_quad_schedule_plan(monkeypatch):
    """The four-wave (quad) schedule is never the library's own choice; forced, it applies to
    W8A8 only and the other modes run plain (host query, no GPU)."""
    from m5kernels_amd.hip import launch_override, launch_plan

    for shape in ((4096, 4096), (9914, 4096), (4096, 7168)):
        assert launch_plan("int8", *shape, 256)[0] != "quad"
    with launch_override("quad"):
        assert launch_plan("int8", 9914, 4096, 256) == ("quad", -1)
        assert launch_plan("bf16", 4096, 7168, 256) == ("plain", -1)
        assert launch_plan("fp8", 4096, 4096, 256) == ("plain", -1)
    monkeypatch.setenv("M5K_GEMM_SCHEDULE", "quad")
    assert launch_plan("int8", 4096, 7168, 256) == ("quad", -1)
    assert launch_plan("fp32", 9914, 4096, 256) == ("plain", -1)


def test_tail_split_plan_decisions():
    """Host schedule of the W8A8 linear on 256 CUs: the row split is taken where the measured
    cost model says it pays (H3 widths at M 4096) and declined where it does not (M 9914 x
    4096 x 4096, short K, tails over half a round, whole rounds, few-tile shapes)."""
    from m5kernels_amd.hip import splitk_plan, tail_split_plan

    assert tail_split_plan(4096, 5376, 5376) == (3072, 3)
    assert tail_split_plan(4096, 5376, 14336) == (3072, 3)
    assert tail_split_plan(4352, 4096, 2048) == (4096, 4)
    for shape in [(9914, 4096, 4096), (4096, 5376, 2048), (4096, 14336, 5376), (4096, 7168, 5376),
                  (4096, 4096, 16384), (1024, 5376, 5376)]:
        assert tail_split_plan(*shape) is None, shape
    # Above M = 768 the plain launch (mixed / narrow tiles) measured faster than any split,
    # except for narrow outputs whose few tiles leave most CUs idle.
    assert splitk_plan(1024, 5376, 5376) == 1 and splitk_plan(1024, 4096, 4096) == 1
    assert splitk_plan(1024, 96, 5376) == 2 and splitk_plan(1024, 32, 5376) == 2
    # ... and for long K when the tiles fill under 3/8 of the CUs: whole-tile K ranges fill the
    # chip (M 1024 at N 5376 / 4096 and K 14336 / 16384); M 1536 and up keeps the plain launch.
    assert splitk_plan(1024, 5376, 14336) == 3 and splitk_plan(1024, 4096, 16384) == 4
    assert splitk_plan(1536, 5376, 14336) == 1 and splitk_plan(2048, 4096, 16384) == 1
    assert splitk_plan(1024, 5376, 14336, skinny=False) == 3
    # Two tile rows: 256 x 64 split tiles while 2 * ceil(N / 64) * splits fits one round.
    assert splitk_plan(512, 4096, 4096) == 2 and splitk_plan(512, 1536, 5376) == 5
    # One tile row, K <= 8192: split counts sized to 256 x 64 tiles (64 columns at N 4096).
    assert splitk_plan(128, 4096, 4096) == 4 and splitk_plan(1, 4096, 4096) == 4
    assert splitk_plan(128, 7168, 5376) == 2 and splitk_plan(128, 1536, 5376) == 10
    # 224 columns of 64 need two rounds even at 2 splits: 256 x 128 tiles (112 columns) take
    # them, and K > 8192 goes straight to 256 x 128 tiles.
    assert splitk_plan(128, 14336, 5376) == 2 and splitk_plan(128, 5376, 14336) == 6
    assert splitk_plan(128, 4096, 16384) == 8
    # 448 columns of 128 still need two rounds: 256 x 256 tiles with the general rule.
    assert splitk_plan(128, 28672, 5376) == 2
    for m in range(256, 12000, 397):
        for n in (1536, 4096, 5120, 5376, 7168):
            plan = tail_split_plan(m, n, 4096)
            if plan is None:
                continue
            rows, splits = plan
            tiles_n = -(-n // 256)
            assert rows % 256 == 0 and 0 < rows < m and 2 <= splits <= 16
            assert (rows // 256) * tiles_n <= ((-(-m // 256) * tiles_n) // 256) * 256
            assert (-(-(m - rows) // 256)) * tiles_n * splits <= 256
