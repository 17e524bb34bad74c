"""Per-op experiment preparation for ``run_case``: seeded inputs, the op under test on the GPU,
and bounded float64 references with the reference's gates.

Every ``prepare_*`` returns ``(fn, check, expected, original, stages, meta)``:
``fn`` runs the resident-input computation, ``check`` extracts the sampled outputs as float64,
``expected`` is the float64 result of the decoded operands (implementation gate), ``original``
the float64 result of the unquantized inputs (quality gate), ``stages`` named timed sub-steps
(``online_activation_plus_gemm`` is the deployed path: online activation preparation + GEMM),
and ``meta`` the record fields, including ``transform_pass`` for the preparation checks.

Inputs come from ``numpy.random.default_rng(seed)`` in the reference's draw order and are cast
to BF16 by nearest-even on the device, so a seed selects the same data as the reference's
harness.  Backend names are the reference's: "mlx" is the framework baseline (torch / hipBLASLt
on MI355X), "mpp" the native kernels.

Follows engine.prepare_gemm (engine.py:121-244), hadamard_gemm.prepare (hadamard_gemm.py:10-118),
norm_hadamard_gemm.prepare (norm_hadamard_gemm.py:11-484), rms_quant_gemm.prepare
(rms_quant_gemm.py:13-268), gate_epilogue_chain.prepare (gate_epilogue_chain.py:13-288) and
qk_rope_experiment.prepare (qk_rope_experiment.py:13-294).
"""

from __future__ import annotations

import hashlib
from numbers import Integral, Real

import numpy as np
import torch
import torch.nn.functional as F

from .. import (
    fused_gated_residual_norm_hadamard_quantize,
    fused_norm_hadamard_quantize,
    gated_residual_add,
    gemm,
    norm_shift_split_gemm,
    projection_qk_rope,
    qk_norm_rope,
    quantize,
    rms_quantize,
    rotate,
    rotate_quantize,
    shift_split_condition,
    unfused_norm,
)
from . import numerics as nx
from .engine import NumericalMismatch, all_finite

BF = torch.bfloat16
FLOAT_DTYPES = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}
DISTRIBUTIONS = ("normal", "outliers", "zeros")


def _dev(a, dtype=BF):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to("cuda").to(dtype)


def _idx(i):
    return torch.as_tensor(np.asarray(i), device="cuda", dtype=torch.long)


def _f64(t):
    return t.float().cpu().numpy().astype(np.float64)


def _rows(t, ri):
    return _f64(t.index_select(0, _idx(ri)))


def _grid(t, ri, ci):
    return _f64(t.index_select(0, _idx(ri)).index_select(1, _idx(ci)))


def _outliers(t, period):
    factor = torch.where(torch.arange(t.shape[-1], device=t.device) % period == 0, 20, 1)
    return (t * factor).to(t.dtype)


def _dtype_name(t):
    return str(t.dtype).replace("torch.", "")


def _decoded(q, s, mode, rows):
    return nx.dequantize(q.index_select(0, _idx(rows)).cpu().numpy(), s.index_select(0, _idx(rows)).cpu().numpy(),
                         mode)


def _positive_int(value):
    return not isinstance(value, bool) and isinstance(value, Integral) and value > 0


# ---- GEMM (engine.py:121-244) ------------------------------------------------------------------


def prepare_gemm(c, backend, precision, seed, distribution, tile):
    m, n, k = c["m"], c["n"], c["k"]
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((m, k), dtype=np.float32)
    b = rng.standard_normal((n, k), dtype=np.float32) / np.sqrt(k)
    if distribution == "outliers":
        a[:, ::127] *= 20
        b[:, ::131] *= 20
    elif distribution == "zeros":
        a.fill(0)
        b.fill(0)
    dtype = FLOAT_DTYPES.get(precision, BF)
    x, w = _dev(a, dtype), _dev(b, dtype)
    ri, ci = nx.sample_indices(m), nx.sample_indices(n)
    original = _rows(x, ri) @ _rows(w, ci).T
    expected = original
    stages = {}
    quant = False
    if backend == "mpp-hadamard":
        return _prepare_hadamard_gemm(c, x, w, ri, ci, original, precision, tile)
    if backend == "mlx":
        if precision not in FLOAT_DTYPES:
            raise NotImplementedError("the framework baseline uses floating point operands; no A8 claim")

        def fn():
            return F.linear(x, w)

        path = "torch.nn.functional.linear (hipBLASLt)"
    elif backend in ("mpp", "mx-emulated"):
        if backend == "mx-emulated" and precision != "mxint8":
            raise NotImplementedError("mx-emulated is only for MXINT8")
        if precision in FLOAT_DTYPES:

            def fn():
                return gemm(x, w, precision, tile, output_dtype=dtype)

            path = f"m5k_gemm_float ({precision} MFMA, FP32 accumulation)"
        elif precision in ("int8", "fp8", "mxint8"):
            aq, sa = quantize(x, precision)
            bq, sb = quantize(w, precision)
            torch.cuda.synchronize()
            expected = _decoded(aq, sa, precision, ri) @ _decoded(bq, sb, precision, ci).T

            def fn():
                return gemm(aq, bq, precision, tile, a_scales=sa, b_scales=sb, output_dtype=dtype)

            def online():
                q, s = quantize(x, precision, tag="online")
                return gemm(q, bq, precision, tile, a_scales=s, b_scales=sb, output_dtype=dtype)

            stages = {"activation_quantization": lambda: quantize(x, precision, tag="stage"),
                      "online_activation_plus_gemm": online}
            path = {"int8": "m5k_gemm_i8 (i8 MFMA, INT32 accumulation)",
                    "fp8": "m5k_gemm_f8 (OCP E4M3 MFMA, FP32 accumulation)",
                    "mxint8": "exact MXINT8 to BF16 expansion, then BF16 MFMA"}[precision]
            quant = True
        else:
            raise ValueError(precision)
    else:
        raise NotImplementedError(f"GEMM backend {backend} is not implemented")

    def check(y):
        return _grid(y, ri, ci)

    meta = dict(
        compute_path=path,
        input_dtype=_dtype_name(x),
        output_dtype=_dtype_name(x),
        reference="NumPy float64 sampled rows x columns, full K",
        sample_rows=ri.tolist(),
        sample_cols=ci.tolist(),
        quantization="symmetric_per_token_A_per_output_channel_W" if quant and precision != "mxint8" else precision,
        weight_quantization_timed=False,
        weight_layout="N,K; transpose in matmul",
        mac_operations=2 * m * n * k,
        bytes_lower_bound=(m * k + n * k) * (1 if quant else (4 if precision == "fp32" else 2))
        + m * n * (4 if precision == "fp32" else 2),
    )
    return fn, check, expected, original, stages, meta


def _prepare_hadamard_gemm(c, x, w, ri, ci, original, precision, tile):
    """Online X D H + quantize before the W8A8/FP8 GEMM; W rotated offline (hadamard_gemm.py:10-118)."""
    if precision not in ("int8", "fp8"):
        raise NotImplementedError("mpp-hadamard supports INT8 and FP8 with BF16 output")
    config = c.get("hadamard", {})
    block = config.get("block_size", 256)
    sign_seed = config.get("sign_seed")
    implementation = config.get("implementation", "metal")
    m, k = x.shape
    n = w.shape[0]
    signs_np = nx.hadamard_signs(k, sign_seed) if sign_seed is not None else np.ones(k, np.int8)
    signs = torch.from_numpy(signs_np).to("cuda")

    def rotation(z):
        return rotate(z, block, signs, implementation=implementation)

    xr, wr = rotation(x), rotation(w)
    ref_a = nx.block_hadamard(_rows(x, ri), block, signs_np)
    ref_w = nx.block_hadamard(_rows(w, ci), block, signs_np)
    error_a, error_w = nx.metrics(_rows(xr, ri), ref_a), nx.metrics(_rows(wr, ci), ref_w)
    dot_error = nx.metrics(ref_a @ ref_w.T, original)
    rotation_finite = all_finite((xr, wr))
    transform_pass = bool(rotation_finite and nx.passes(error_a, 1e-5) and nx.passes(error_w, 1e-5)
                          and nx.passes(dot_error, 1e-12))
    aq, sa = quantize(xr, precision, tag="hadamard_packed")
    bq, sb = quantize(wr, precision, tag="hadamard_packed")
    torch.cuda.synchronize()
    expected = _decoded(aq, sa, precision, ri) @ _decoded(bq, sb, precision, ci).T
    rotated_dot = _rows(xr, ri) @ _rows(wr, ci).T

    def compute(q, scale):
        return gemm(q, bq, precision, tile, a_scales=scale, b_scales=sb, output_dtype=BF)

    def online_prepare():
        # INT8: the rotation and quantizer in one dispatch (the codes and scales of
        # quantize(rotate(x))); FP8 keeps the two.  The stages above time the halves one by one.
        if precision == "int8":
            return rotate_quantize(x, block, signs)
        return quantize(rotation(x), precision, tag="hadamard_online")

    stages = {
        "activation_hadamard": lambda: rotation(x),
        "activation_quantization": lambda: quantize(xr, precision, tag="hadamard_stage"),
        "activation_hadamard_plus_quantization": online_prepare,
        "online_activation_plus_gemm": lambda: compute(*online_prepare()),
    }
    meta = dict(
        compute_path="block_hadamard_then_mfma_" + precision,
        online_activation_preparation=("block Hadamard and INT8 in one dispatch (the codes and scales of "
                                       "quantize(rotate(x)))" if precision == "int8" else
                                       "block Hadamard, then the FP8 quantizer"),
        input_dtype=_dtype_name(x),
        rotated_dtype="float32",
        output_dtype="bfloat16",
        reference="NumPy float64 original/decoded dot products, sampled rows x columns, full K",
        sample_rows=ri.tolist(),
        sample_cols=ci.tolist(),
        quantization="symmetric_per_token_rotated_A_per_output_channel_rotated_W",
        weight_quantization_timed=False,
        weight_rotation_timed=False,
        weight_layout="N,K; identically right-rotated before quantization; transpose in matmul",
        mac_operations=2 * m * n * k,
        bytes_lower_bound=m * k + n * k + m * n * 2,
        bytes_lower_bound_scope="prequantized GEMM only; excludes rotation/quantization traffic",
        decoded_quantization_error=nx.metrics(expected, rotated_dot),
        actual_rotation_dot_error=nx.metrics(rotated_dot, original),
        transform_pass=transform_pass,
        transform=dict(
            kind="normalized_block_sylvester_hadamard",
            block_size=block,
            implementation=implementation,
            sign_seed=sign_seed,
            sign_rng="NumPy PCG64" if sign_seed is not None else "all +1",
            sign_sha256=hashlib.sha256(signs_np.tobytes()).hexdigest(),
            ordering="X D H; identical fixed D and H for activation and weight",
            padding=0,
            online_timing_includes="BF16 input to FP32 rotation, quantization, GEMM, BF16 output",
            activation_error=error_a,
            weight_error=error_w,
            float64_dot_preservation_error=dot_error,
            all_rotated_values_finite=rotation_finite,
            implementation_relative_l2_limit=1e-5,
            dot_preservation_relative_l2_limit=1e-12,
        ),
    )
    return (lambda: compute(aq, sa)), (lambda y: _grid(y, ri, ci)), expected, original, stages, meta


# ---- Norm / gated residual + H + INT8 before a GEMM (norm_hadamard_gemm.py:11-484) ------------

NORM_BACKENDS = {("norm-staged", "int8"), ("norm-fused", "int8"), ("norm-shift-split", "int8"), ("mlx", "bf16")}
GATED_BACKENDS = {("residual-separate", "int8"), ("residual-fused", "int8"), ("mlx", "bf16")}


def prepare_norm_hadamard_gemm(c, backend, precision, seed, distribution, tile):
    gated = c["op"] == "gated_norm_hadamard_gemm"
    allowed = GATED_BACKENDS if gated else NORM_BACKENDS
    if (backend, precision) not in allowed:
        raise NotImplementedError(f"supported backend/precision pairs: {sorted(allowed)}")
    m, n, k = c["m"], c["n"], c["k"]
    cfg = c.get("fusion", {})
    norm, eps = cfg.get("norm", "rms"), cfg.get("epsilon", 1e-5)
    block, threads = cfg.get("block_size", 256), cfg.get("threads", 256)
    passes, rounding = cfg.get("passes", "one_read"), cfg.get("round_output", "input")
    sign_seed = cfg.get("sign_seed")
    split_shift = backend == "norm-shift-split"
    bias_backend = cfg.get("bias_backend", "mlx-fp32-convert")
    if split_shift and (norm != "rms" or rounding != "fp32"):
        raise NotImplementedError("shift splitting requires RMS and round_output=fp32")
    if split_shift and passes != "one_read":
        raise NotImplementedError("shift splitting supports only passes=one_read")
    if split_shift and bias_backend not in ("mlx-fp32-convert", "mpp-bf16-to-fp32"):
        raise NotImplementedError("unsupported bias preparation backend")
    rng = np.random.default_rng(seed)
    x = _dev(rng.standard_normal((m, k), dtype=np.float32))
    w = _dev(rng.standard_normal((n, k), dtype=np.float32))
    if distribution == "zeros":
        x, w = torch.zeros_like(x), torch.zeros_like(w)
    elif distribution == "outliers":
        x, w = _outliers(x, 127), _outliers(w, 131)
    gamma = _dev(1 + 0.1 * rng.standard_normal(k).astype(np.float32))
    scale = _dev(0.2 * rng.standard_normal(k).astype(np.float32))
    shift = _dev(0.1 * rng.standard_normal(k).astype(np.float32))
    signs_np = nx.hadamard_signs(k, sign_seed) if sign_seed is not None else np.ones(k, np.int8)
    signs = torch.from_numpy(signs_np).to("cuda")
    ri, ci = nx.sample_indices(m), nx.sample_indices(n)
    branch = gate = None
    if gated:
        branch = _dev(rng.standard_normal((m, k), dtype=np.float32))
        gate = _dev(0.2 * rng.standard_normal(k).astype(np.float32))
        if distribution == "zeros":
            branch = torch.zeros_like(branch)
        elif distribution == "outliers":
            branch = _outliers(branch, 137)
        ideal_residual = _rows(x, ri) + _rows(branch, ri) * _f64(gate)
        ref_residual = nx.bf16_round(ideal_residual)
    else:
        ref_residual = _rows(x, ri)
    g64, sc64, sh64 = _f64(gamma), _f64(scale), _f64(shift)
    ref_norm = nx.norm_modulate(ref_residual, g64, sc64, sh64, norm=norm, eps=eps)
    rounded_ref = nx.bf16_round(ref_norm) if rounding == "input" else ref_norm.astype(np.float32).astype(np.float64)
    ref_w = _rows(w, ci)
    # The split policy is defined before any intermediate dtype round (norm_hadamard_gemm.py:100-103).
    original = (ref_norm if split_shift else rounded_ref) @ ref_w.T

    def residual_only():
        return gated_residual_add(x, branch, gate, threads=threads) if gated else x

    def norm_only():
        return unfused_norm(residual_only(), gamma, scale, shift, norm=norm, epsilon=eps, round_output=rounding,
                            threads=threads)

    def check(y):
        if gated:
            y, updated = y
            actual_residual = _rows(updated, ri)
            if not np.array_equal(actual_residual, ref_residual):
                raise NumericalMismatch("updated residual differs from independently rounded BF16 reference",
                                        residual_update_error=nx.metrics(actual_residual, ref_residual),
                                        residual_update_exact_match=False)
        return _grid(y, ri, ci)

    meta = dict(
        compute_path=(("gate_norm_then_torch_bf16_gemm" if gated else "norm_then_torch_bf16_gemm")
                      if backend == "mlx" else backend),
        input_dtype="bfloat16",
        output_dtype="bfloat16",
        mac_operations=2 * m * n * k,
        reference="NumPy float64 normalization/rotation/dots; sampled rows/columns, full K",
        sample_rows=ri.tolist(),
        sample_cols=ci.tolist(),
        norm=norm,
        epsilon=eps,
        modulation="per-channel gamma, scale and shift shared by all rows",
        normalization_rounding=rounding,
        rounding_contract=("FP32 norm and modulation, then one input-dtype round before rotation"
                           if rounding == "input" else "FP32 norm, modulation and rotation; no BF16 intermediate"),
        ideal_normalization_rounding_error=nx.metrics(rounded_ref, ref_norm),
        weight_rotation_timed=False,
        weight_quantization_timed=False,
    )
    if gated:
        meta.update(
            gated_residual=True,
            residual_contract="BF16(float32(R) + float32(branch)*float32(gate)); no BF16 product round",
            residual_output_timed_stages=["activation_prepare", "online_activation_plus_gemm"],
            prequantized_timing_reuses_resident_residual=True,
            residual_output_dtype="bfloat16",
            residual_input_mutated=False,
            gate="per-channel signed gate shared by rows; independent of upcoming modulation",
            ideal_residual_rounding_error=nx.metrics(ref_residual, ideal_residual),
        )
    if backend == "mlx":

        def baseline():
            updated = residual_only()
            normalized = unfused_norm(updated, gamma, scale, shift, norm=norm, epsilon=eps, round_output=rounding,
                                      threads=threads)
            y = F.linear(normalized, w.to(normalized.dtype)).to(BF)
            return (y, updated) if gated else y

        updated0 = residual_only()
        normalized0 = unfused_norm(updated0, gamma, scale, shift, norm=norm, epsilon=eps, round_output=rounding,
                                   threads=threads)
        w_cast = w.to(normalized0.dtype)

        def fn():
            y = F.linear(normalized0, w_cast).to(BF)
            return (y, updated0) if gated else y

        def prepare_baseline():
            updated = residual_only()
            normalized = unfused_norm(updated, gamma, scale, shift, norm=norm, epsilon=eps, round_output=rounding,
                                      threads=threads)
            return (normalized, updated) if gated else normalized

        return fn, check, original, original, {"activation_prepare": prepare_baseline,
                                                "online_activation_plus_gemm": baseline}, meta

    if split_shift:
        combined, projected_bias = shift_split_condition(gamma, scale, shift, w, bias_backend=bias_backend)

    def activation():
        if split_shift:
            return rms_quantize(x, combined, signs, block, threads=threads, fold_scale=True, epsilon=eps)
        if gated:
            if backend == "residual-fused":
                return fused_gated_residual_norm_hadamard_quantize(
                    x, branch, gate, gamma, scale, shift, signs, block, norm=norm, epsilon=eps,
                    round_output=rounding, threads=threads, passes=passes)
            updated = residual_only()
            q, s = fused_norm_hadamard_quantize(updated, gamma, scale, shift, signs, block, norm=norm, epsilon=eps,
                                                round_output=rounding, threads=threads, passes=passes)
            return q, s, updated
        if backend == "norm-fused":
            return fused_norm_hadamard_quantize(x, gamma, scale, shift, signs, block, norm=norm, epsilon=eps,
                                                round_output=rounding, threads=threads, passes=passes)
        return quantize(rotate(norm_only(), block, signs), "int8", tag="norm_staged")

    prepared = activation()
    aq, sa = prepared[:2]
    torch.cuda.synchronize()
    residual_pass = True
    if gated:
        actual_residual = _rows(prepared[2], ri)
        residual_pass = bool(np.array_equal(actual_residual, ref_residual) and all_finite(prepared[2]))
        meta["residual_update_error"] = nx.metrics(actual_residual, ref_residual)
        meta["residual_update_exact_match"] = residual_pass
    rotated_w = rotate(w, block, signs)
    bq, sb = quantize(rotated_w, "int8", tag="norm_offline_weight")
    torch.cuda.synchronize()
    actual_a = _decoded(aq, sa, "int8", ri)
    actual_w = _decoded(bq, sb, "int8", ci)
    activation_ref = ref_norm - sh64 if split_shift else rounded_ref
    ref_rotated = nx.block_hadamard(activation_ref, block, signs_np)
    ref_rotated_w = nx.block_hadamard(ref_w, block, signs_np)
    ref_q, ref_scale, ref_decoded = nx.symmetric_int8(ref_rotated)
    ref_w_q, ref_w_scale, ref_w_decoded = nx.symmetric_int8(ref_rotated_w)
    weight_rotation_error = nx.metrics(_rows(rotated_w, ci), ref_rotated_w)
    weight_error = nx.metrics(actual_w, ref_w_decoded)
    weight_scale_error = nx.metrics(_rows(sb[:, None], ci)[:, 0], ref_w_scale)
    weight_max_code_error = float(np.max(np.abs(_rows(bq, ci) - ref_w_q)))
    activation_error = nx.metrics(actual_a, ref_decoded)
    scale_error = nx.metrics(_rows(sa[:, None], ri)[:, 0], ref_scale)
    reference_bias = sh64 @ ref_w.T if split_shift else 0
    dot_error = nx.metrics(ref_rotated @ ref_rotated_w.T + reference_bias, original)
    max_code_error = float(np.max(np.abs(_rows(aq, ri) - ref_q)))
    finite = bool(all_finite((sa, sb, rotated_w)) and (sa > 0).all().item() and (sb > 0).all().item())
    expected = actual_a @ actual_w.T
    if split_shift:
        actual_bias = _f64(projected_bias)[ci]
        bias_error = nx.metrics(actual_bias, reference_bias)
        finite = finite and all_finite(projected_bias) and nx.passes(bias_error, 1e-5)
        expected = expected + actual_bias
        meta.update(
            shift_split=True,
            shift_projection_policy="original BF16 weights, FP32 bias; main GEMM uses INT8 weights",
            shift_projection_error=bias_error,
            condition_rows=1,
            bias_preparation_backend=bias_backend,
            condition_prepare_timed=True,
            condition_prepare_in_online_activation_plus_gemm=False,
            conditioning_inclusive_stage="online_with_conditioning",
            retained_original_bf16_weights_for_bias=True,
            native_bf16_boundary_diagnostic=nx.metrics(nx.bf16_round(ref_norm) @ ref_w.T, original),
        )
    activation_scale_limit = 1e-5 if split_shift else 0.008
    meta.update(
        quantization="symmetric_per_token_rotated_A_per_output_channel_rotated_W",
        transform_pass=bool(
            finite and residual_pass and nx.passes(activation_error, 0.008)
            and nx.passes(scale_error, activation_scale_limit) and max_code_error <= 1
            and nx.passes(weight_rotation_error, 1e-5) and nx.passes(weight_error, 0.008)
            and nx.passes(weight_scale_error, 1e-5) and weight_max_code_error <= 1 and nx.passes(dot_error, 1e-12)
        ),
        activation_implementation_error=activation_error,
        activation_scale_error=scale_error,
        activation_scale_relative_l2_limit=activation_scale_limit,
        activation_max_code_difference=max_code_error,
        activation_implementation_relative_l2_limit=0.008,
        activation_max_code_difference_limit=1,
        weight_rotation_error=weight_rotation_error,
        weight_implementation_error=weight_error,
        weight_scale_error=weight_scale_error,
        weight_max_code_difference=weight_max_code_error,
        activation_preparation_total_error=nx.metrics(actual_a, ref_rotated),
        decoded_preparation_total_error=nx.metrics(expected, original),
        ideal_activation_quantization_error=nx.metrics(ref_decoded, ref_rotated),
        ideal_decoded_quantization_error=nx.metrics(ref_decoded @ ref_w_decoded.T + reference_bias, original),
        transform=dict(
            kind="normalized_block_sylvester_hadamard",
            block_size=block,
            implementation=backend,
            sign_seed=sign_seed,
            sign_sha256=hashlib.sha256(signs_np.tobytes()).hexdigest(),
            float64_dot_preservation_error=dot_error,
            threads=threads,
            passes=passes,
        ),
    )

    def compute(q, s):
        if split_shift:
            return gemm(q, bq, "int8", tile, a_scales=s, b_scales=sb, output_dtype=BF, bias=projected_bias)
        return gemm(q, bq, "int8", tile, a_scales=s, b_scales=sb, output_dtype=BF)

    def fn():
        y = compute(aq, sa)
        return (y, prepared[2]) if gated else y

    def online():
        packed = activation()
        y = compute(*packed[:2])
        return (y, packed[2]) if gated else y

    stages = {"activation_prepare": activation, "online_activation_plus_gemm": online}
    if split_shift:

        def condition_prepare():
            return shift_split_condition(gamma, scale, shift, w, bias_backend=bias_backend)

        def online_with_conditioning():
            comb, bias = condition_prepare()
            return norm_shift_split_gemm(x, bq, sb, signs, comb, bias, block, epsilon=eps, threads=threads)

        complete = online_with_conditioning()
        torch.cuda.synchronize()
        complete_error = nx.metrics(_grid(complete, ri, ci), expected)
        meta["conditioning_inclusive_implementation_error"] = complete_error
        meta["transform_pass"] = bool(meta["transform_pass"] and nx.passes(complete_error, 0.008)
                                      and all_finite(complete))
        stages.update(condition_prepare=condition_prepare, online_with_conditioning=online_with_conditioning)
    return fn, check, expected, original, stages, meta


# ---- RMS scale-folded INT8 + GEMM (rms_quant_gemm.py:13-268) ------------------------------------


def validate_rms_config(c, backend, precision, distribution):
    """Reject unsupported semantics before any device work (rms_quant_gemm.py:13-62)."""
    if (backend, precision) not in {("rms-direct", "int8"), ("rms-folded", "int8")}:
        raise NotImplementedError("rms_quant_gemm supports rms-direct/rms-folded with INT8 only")
    if c.get("op") != "rms_quant_gemm":
        raise ValueError("operation must be rms_quant_gemm")
    forbidden = {"shift", "norm", "round_output"}.intersection(c)
    if forbidden:
        raise NotImplementedError(f"unsupported RMS semantics options: {sorted(forbidden)}")
    for key in ("m", "n", "k"):
        if not _positive_int(c.get(key)):
            raise ValueError(f"{key} must be a positive integer")
    cfg = c.get("rms_quant", {})
    if not isinstance(cfg, dict):
        raise ValueError("rms_quant must be a configuration object")
    unknown = set(cfg) - {"block_size", "gamma", "threads", "epsilon", "sign_seed"}
    if unknown:
        raise NotImplementedError(f"unsupported rms_quant options: {sorted(unknown)}; "
                                  "this experiment requires RMS, zero shift and no BF16 intermediate")
    config = dict(block_size=1, gamma="identity", threads=256, epsilon=1e-5, sign_seed=None)
    config.update(cfg)
    block = config["block_size"]
    if not _positive_int(block):
        raise ValueError("block_size must be a positive integer")
    if block not in (1, 256):
        raise NotImplementedError("rms_quant_gemm supports block_size 1 or 256")
    if c["k"] % block:
        raise NotImplementedError("K must be divisible by block_size; padding is not implicit")
    if config["gamma"] not in ("identity", "random"):
        raise NotImplementedError("gamma must be identity or random")
    threads = config["threads"]
    if isinstance(threads, bool) or not isinstance(threads, Integral):
        raise ValueError("threads must be an integer")
    if threads not in (128, 256, 512):
        raise NotImplementedError("supported threadgroup sizes are 128, 256 and 512")
    eps = config["epsilon"]
    if isinstance(eps, bool) or not isinstance(eps, Real) or not np.isfinite(eps) or eps <= 0:
        raise ValueError("epsilon must be positive and finite")
    with np.errstate(over="ignore", under="ignore"):
        eps32 = np.float32(eps)
    if not np.isfinite(eps32) or eps32 <= 0:
        raise ValueError("epsilon must remain positive and finite in float32")
    seed = config["sign_seed"]
    if seed is not None and (isinstance(seed, bool) or not isinstance(seed, Integral) or seed < 0):
        raise ValueError("sign_seed must be a nonnegative integer or null")
    if distribution not in DISTRIBUTIONS:
        raise ValueError("distribution must be normal, outliers or zeros")
    return config


def prepare_rms_quant_gemm(c, backend, precision, seed, distribution, tile):
    cfg = validate_rms_config(c, backend, precision, distribution)
    m, n, k = c["m"], c["n"], c["k"]
    block, threads, eps, sign_seed = cfg["block_size"], cfg["threads"], cfg["epsilon"], cfg["sign_seed"]
    fold = backend == "rms-folded"
    rng = np.random.default_rng(seed)
    x = _dev(rng.standard_normal((m, k), dtype=np.float32))
    w = _dev(rng.standard_normal((n, k), dtype=np.float32))
    if distribution == "zeros":
        x, w = torch.zeros_like(x), torch.zeros_like(w)
    elif distribution == "outliers":
        x, w = _outliers(x, 127), _outliers(w, 131)
    gamma_np = (1 + 0.2 * rng.standard_normal(k).astype(np.float32) if cfg["gamma"] == "random"
                else np.ones(k, np.float32))
    gamma = torch.from_numpy(gamma_np).to("cuda")
    signs_np = nx.hadamard_signs(k, sign_seed) if sign_seed is not None else np.ones(k, np.int8)
    signs = torch.from_numpy(signs_np).to("cuda")
    ri, ci = nx.sample_indices(m), nx.sample_indices(n)
    ref_x, ref_w = _rows(x, ri), _rows(w, ci)
    ref_a = nx.rms_quantize(ref_x, gamma_np, signs_np, block, eps=eps)
    ref_norm = ref_x * ref_a["inverse_rms"][:, None] * gamma_np.astype(np.float64)
    original = ref_norm @ ref_w.T
    ref_rotated_w = nx.block_hadamard(ref_w, block, signs_np)
    ref_w_q, ref_w_scale, ref_w_decoded = nx.symmetric_int8(ref_rotated_w)

    def weight_transform():
        if block == 1:
            dense = w.float()
            return dense * signs.float() if sign_seed is not None else dense
        return rotate(w, block, signs)

    def activation(tag="rms_online"):
        return rms_quantize(x, gamma, signs, block, threads=threads, fold_scale=fold, epsilon=eps, tag=tag)

    aq, sa = activation("rms_packed")
    rotated_w = weight_transform()
    bq, sb = quantize(rotated_w, "int8", tag="rms_weight_packed")
    torch.cuda.synchronize()
    actual_a = _decoded(aq, sa, "int8", ri)
    actual_w = _decoded(bq, sb, "int8", ci)
    expected = actual_a @ actual_w.T
    activation_error = nx.metrics(actual_a, ref_a["dequantized"])
    scale_error = nx.metrics(_rows(sa[:, None], ri)[:, 0], ref_a["scales"])
    max_code_error = float(np.max(np.abs(_rows(aq, ri) - ref_a["quantized"])))
    weight_rotation_error = nx.metrics(_rows(rotated_w, ci), ref_rotated_w)
    weight_error = nx.metrics(actual_w, ref_w_decoded)
    weight_scale_error = nx.metrics(_rows(sb[:, None], ci)[:, 0], ref_w_scale)
    weight_max_code_error = float(np.max(np.abs(_rows(bq, ci) - ref_w_q)))
    dot_error = nx.metrics(ref_a["normalized_rotated"] @ ref_rotated_w.T, original)
    finite = bool(all_finite((sa, sb, rotated_w)) and (sa > 0).all().item() and (sb > 0).all().item()
                  and (aq >= -127).all().item() and (bq >= -127).all().item())
    transform_pass = bool(
        finite and nx.passes(activation_error, 0.008) and nx.passes(scale_error, 1e-5) and max_code_error <= 1
        and nx.passes(weight_rotation_error, 1e-5) and nx.passes(weight_error, 0.008)
        and nx.passes(weight_scale_error, 1e-5) and weight_max_code_error <= 1 and nx.passes(dot_error, 1e-12)
    )
    rounded_norm = nx.bf16_round(ref_norm)
    rounded_rotated = nx.block_hadamard(rounded_norm, block, signs_np)

    def compute(q, s):
        return gemm(q, bq, "int8", tile, a_scales=s, b_scales=sb, output_dtype=BF)

    meta = dict(
        compute_path=backend,
        input_dtype="bfloat16",
        output_dtype="bfloat16",
        preparation_dtype="float32",
        mac_operations=2 * m * n * k,
        reference="NumPy float64 RMS/gamma/rotation/dots; sampled rows/columns, full K",
        sample_rows=ri.tolist(),
        sample_cols=ci.tolist(),
        norm="rms",
        epsilon=eps,
        gamma=cfg["gamma"],
        gamma_sha256=hashlib.sha256(gamma_np.tobytes()).hexdigest(),
        fold_scale=fold,
        additive_shift=False,
        normalization_rounding="fp32",
        rounding_contract="FP32 RMS and gamma/rotation; no BF16 intermediate; BF16 GEMM output",
        quantization="symmetric_per_token_rotated_A_per_output_channel_rotated_W",
        weight_preparation_in_online=False,
        weight_preparation_timed=True,
        weight_preparation_timing_stage="offline_weight_prepare",
        all_preparation_values_finite=finite,
        transform_pass=transform_pass,
        activation_implementation_error=activation_error,
        activation_scale_error=scale_error,
        activation_max_code_difference=max_code_error,
        activation_implementation_relative_l2_limit=0.008,
        activation_scale_relative_l2_limit=1e-5,
        activation_max_code_difference_limit=1,
        weight_rotation_error=weight_rotation_error,
        weight_implementation_error=weight_error,
        weight_scale_error=weight_scale_error,
        weight_max_code_difference=weight_max_code_error,
        activation_preparation_total_error=nx.metrics(actual_a, ref_a["normalized_rotated"]),
        ideal_activation_quantization_error=nx.metrics(ref_a["dequantized"], ref_a["normalized_rotated"]),
        decoded_preparation_total_error=nx.metrics(expected, original),
        ideal_decoded_quantization_error=nx.metrics(ref_a["dequantized"] @ ref_w_decoded.T, original),
        bf16_intermediate_diagnostic=dict(
            diagnostic_only=True,
            contract="hypothetical BF16 round after RMS*gamma, before D*H; not executed",
            normalization_error=nx.metrics(rounded_norm, ref_norm),
            rotated_error=nx.metrics(rounded_rotated, ref_a["normalized_rotated"]),
            gemm_difference=nx.metrics(rounded_norm @ ref_w.T, original),
        ),
        transform=dict(
            kind="signed_identity" if block == 1 else "normalized_block_sylvester_hadamard",
            block_size=block,
            sign_seed=sign_seed,
            sign_sha256=hashlib.sha256(signs_np.tobytes()).hexdigest(),
            float64_dot_preservation_error=dot_error,
            threads=threads,
        ),
    )
    stages = dict(
        activation_prepare=lambda: activation("rms_stage"),
        online_activation_plus_gemm=lambda: compute(*activation()),
        offline_weight_prepare=lambda: quantize(weight_transform(), "int8", tag="rms_weight_stage"),
    )
    return (lambda: compute(aq, sa)), (lambda y: _grid(y, ri, ci)), expected, original, stages, meta


# ---- Gate placement across two projections (gate_epilogue_chain.py:13-288) ---------------------


def _preparation_check(original, rotated, codes, scales, block, rows):
    """Independent sampled-row H256 + INT8 reference with full contraction width."""
    reference = nx.block_hadamard(original, block)
    ref_codes, ref_scale, ref_decoded = nx.symmetric_int8(reference)
    decoded = np.asarray(codes, dtype=np.float64) * np.asarray(scales, dtype=np.float64)[:, None]
    rotation_error = nx.metrics(rotated, reference)
    scale_error = nx.metrics(scales, ref_scale)
    implementation_error = nx.metrics(decoded, ref_decoded)
    code_difference = float(np.max(np.abs(np.asarray(codes, dtype=np.float64) - ref_codes)))
    return dict(
        sample_rows=np.asarray(rows).tolist(),
        reference="independent NumPy float64 H256 and symmetric INT8, sampled rows with full K",
        rotation_error=rotation_error,
        scale_error=scale_error,
        decoded_implementation_error=implementation_error,
        max_code_difference=code_difference,
        ideal_quantization_error=nx.metrics(ref_decoded, reference),
        actual_quantization_total_error=nx.metrics(decoded, reference),
        rotation_relative_l2_limit=1e-5,
        scale_relative_l2_limit=1e-5,
        decoded_implementation_relative_l2_limit=0.008,
        max_code_difference_limit=1,
        passed=bool(nx.passes(rotation_error, 1e-5) and nx.passes(scale_error, 1e-5)
                    and nx.passes(implementation_error, 0.008) and code_difference <= 1),
    )


def prepare_gate_epilogue_chain(c, backend, precision, seed, distribution, tile):
    if backend not in ("gate-in-norm", "gate-in-gemm") or precision != "int8":
        raise NotImplementedError("gate chain uses gate-in-norm/gate-in-gemm with INT8")
    m, h, pk, n = c["m"], c["k"], c["previous_k"], c["n"]
    previous_tile = c.get("previous_tile")
    if previous_tile is None:
        previous_tile = tile
    if not isinstance(previous_tile, (tuple, list)) or len(previous_tile) != 4 or not all(
            _positive_int(v) for v in previous_tile):
        raise ValueError("previous_tile must contain four positive integers")
    previous_tile = tuple(int(v) for v in previous_tile)
    block, threads = 256, 256
    if h % block or pk % block:
        raise NotImplementedError("both K dimensions must divide H256; no implicit padding")
    rng = np.random.default_rng(seed)

    def array(shape, factor=1.0):
        return _dev(rng.standard_normal(shape, dtype=np.float32) * factor)

    x, w0, w1 = array((m, pk)), array((h, pk), pk**-0.5), array((n, h), h**-0.5)
    residual, gate = array((m, h)), array((h,), 0.2)
    gamma = (1 + array((h,), 0.1).float()).to(BF)
    scale, shift = array((h,), 0.2), array((h,), 0.1)
    if distribution == "outliers":
        x, w0, w1 = _outliers(x, 127), _outliers(w0, 131), _outliers(w1, 131)
        residual = _outliers(residual, 137)
    elif distribution == "zeros":
        x, w0, w1, residual = map(torch.zeros_like, (x, w0, w1, residual))
    elif distribution != "normal":
        raise ValueError("unknown distribution")
    signs0 = torch.ones(pk, dtype=torch.int8, device="cuda")
    signs1 = torch.ones(h, dtype=torch.int8, device="cuda")
    ri, ci, wi0 = nx.sample_indices(m), nx.sample_indices(n), nx.sample_indices(h)

    def input_prepare():
        # One dispatch, the same codes and scales as quantize(rotate(x)).
        return rotate_quantize(x, block, signs0)

    rotated_x = rotate(x, block, signs0)
    rotated_w0, rotated_w1 = rotate(w0, block, signs0), rotate(w1, block, signs1)
    aq, sa = quantize(rotated_x, "int8", tag="chain_packed")
    bq0, sb0 = quantize(rotated_w0, "int8", tag="chain_weight0")
    bq1, sb1 = quantize(rotated_w1, "int8", tag="chain_weight1")
    torch.cuda.synchronize()
    rotation_storage_finite = all_finite((rotated_x, rotated_w0, rotated_w1))
    packed_storage_finite = all_finite((sa, sb0, sb1))
    preparation_scales_positive = all(bool((s > 0).all().item()) for s in (sa, sb0, sb1))
    preparation_codes_valid = all(bool((q >= -127).all().item()) for q in (aq, bq0, bq1))
    sampled_rotated_x = _rows(rotated_x, ri)
    sampled_rotated_w0 = _rows(rotated_w0, wi0)
    sampled_rotated_w1 = _rows(rotated_w1, ci)
    del rotated_x, rotated_w0, rotated_w1

    def previous(q, s, fused):
        extra = dict(residual=residual, gate=gate) if fused else {}
        return gemm(q, bq0, "int8", previous_tile, a_scales=s, b_scales=sb0, output_dtype=BF, **extra)

    def transition(z, fused):
        if fused:
            q, s = fused_norm_hadamard_quantize(z, gamma, scale, shift, signs1, threads=threads)
            return q, s, z
        return fused_gated_residual_norm_hadamard_quantize(residual, z, gate, gamma, scale, shift, signs1,
                                                           threads=threads)

    def next_projection(q, s):
        return gemm(q, bq1, "int8", tile, a_scales=s, b_scales=sb1, output_dtype=BF)

    fused = backend == "gate-in-gemm"
    z = previous(aq, sa, fused)
    q1, s1, rnext = transition(z, fused)
    other_z = previous(aq, sa, not fused)
    other_q, other_s, other_r = transition(other_z, not fused)
    torch.cuda.synchronize()
    parity = dict(residual_exact=bool(torch.equal(rnext, other_r)),
                  activation_codes_exact=bool(torch.equal(q1, other_q)),
                  activation_scales_exact=bool(torch.equal(s1, other_s)))
    sampled_r = _rows(rnext, ri)
    actual_a = _decoded(q1, s1, "int8", ri)
    actual_w = _decoded(bq1, sb1, "int8", ci)
    expected = actual_a @ actual_w.T
    rx, rw0, rw1 = _rows(x, ri), _f64(w0), _rows(w1, ci)
    preparation_checks = dict(
        input_activation=_preparation_check(rx, sampled_rotated_x, _rows(aq, ri), _rows(sa[:, None], ri)[:, 0],
                                            block, ri),
        previous_weight=_preparation_check(rw0[wi0], sampled_rotated_w0, _rows(bq0, wi0),
                                           _rows(sb0[:, None], wi0)[:, 0], block, wi0),
        next_weight=_preparation_check(rw1, sampled_rotated_w1, _rows(bq1, ci), _rows(sb1[:, None], ci)[:, 0],
                                       block, ci),
    )
    preparation_pass = bool(rotation_storage_finite and packed_storage_finite and preparation_scales_positive
                            and preparation_codes_valid
                            and all(chk["passed"] for chk in preparation_checks.values()))
    rr, rg = _rows(residual, ri), _f64(gate)
    norm_args = [_f64(v) for v in (gamma, scale, shift)]
    original_branch = nx.bf16_round(rx @ rw0.T)
    original_residual = nx.bf16_round(rr + original_branch * rg)
    original_norm = nx.bf16_round(nx.norm_modulate(original_residual, *norm_args))
    original = original_norm @ rw1.T
    decoded_x = _decoded(aq, sa, "int8", ri)
    decoded_w0 = nx.dequantize(bq0.cpu().numpy(), sb0.cpu().numpy(), "int8")
    decoded_branch = nx.bf16_round(decoded_x @ decoded_w0.T)
    decoded_residual = nx.bf16_round(rr + decoded_branch * rg)
    residual_error = nx.metrics(sampled_r, decoded_residual)
    # The norm/rotation reference takes the actual BF16 residual, separating errors in the
    # previous GEMM from the implementation of the following preparation.
    ref_norm = nx.bf16_round(nx.norm_modulate(sampled_r, *norm_args))
    ref_rot = nx.block_hadamard(ref_norm, block)
    ref_q, ref_scale, ref_decoded = nx.symmetric_int8(ref_rot)
    prep_error = nx.metrics(actual_a, ref_decoded)
    scale_error = nx.metrics(_rows(s1[:, None], ri)[:, 0], ref_scale)
    code_error = float(np.max(np.abs(_rows(q1, ri) - ref_q)))
    finite = bool(all_finite((z, s1, rnext, sb0, sb1)) and (s1 > 0).all().item())
    branch_value = other_z if fused else z
    branch_error = nx.metrics(_rows(branch_value, ri), decoded_branch)
    baseline_residual = _rows(other_r, ri)

    def check(output):
        y, updated = output
        if not np.array_equal(_rows(updated, ri), baseline_residual):
            raise NumericalMismatch("chain residual differs from paired reference path")
        return _grid(y, ri, ci)

    def core(q, s):
        qn, sn, rn = transition(previous(q, s, fused), fused)
        return next_projection(qn, sn), rn

    def offline_weights():
        return (*quantize(rotate(w0, block, signs0), "int8", tag="chain_offline0"),
                *quantize(rotate(w1, block, signs1), "int8", tag="chain_offline1"))

    meta = dict(
        compute_path=backend,
        input_dtype="bf16",
        output_dtype="bf16",
        reference="NumPy float64 full previous projection for sampled rows, next dot full K; explicit BF16 boundaries",
        mac_operations=2 * m * h * pk + 2 * m * n * h,
        sample_rows=ri.tolist(),
        sample_cols=ci.tolist(),
        branch_rounding="BF16 after INT8 dequant, before FP32 gate product",
        residual_rounding="BF16(R + float32(BF16(branch))*float32(gate)); no BF16 product round",
        normalization_rounding="completed AdaLN to BF16 before H256",
        returned_outputs=["next projection", "updated residual"],
        preceding_input_preparation="online H256 and INT8 packing in one dispatch (the codes and scales of quantize(rotate(x)))",
        main_timing_scope="both projections and transition, resident preceding INT8 activation",
        previous_tile=list(previous_tile),
        next_tile=list(tile),
        online_timing_scope="input H/INT8 + previous GEMM + transition + next GEMM + residual output",
        offline_weight_preparation_in_online=False,
        preparation_checks=preparation_checks,
        preparation_rotated_storage_finite=rotation_storage_finite,
        preparation_packed_storage_finite=packed_storage_finite,
        preparation_all_scales_positive=preparation_scales_positive,
        preparation_all_codes_in_symmetric_range=preparation_codes_valid,
        preparation_pass=preparation_pass,
        paired_path_parity=parity,
        previous_branch_implementation_error=branch_error,
        residual_implementation_error=residual_error,
        activation_implementation_error=prep_error,
        activation_scale_error=scale_error,
        activation_max_code_difference=code_error,
        previous_branch_quality_error=nx.metrics(_rows(branch_value, ri), original_branch),
        residual_quality_error=nx.metrics(sampled_r, original_residual),
        activation_quantization_error=nx.metrics(actual_a, ref_rot),
        decoded_chain_quality_error=nx.metrics(expected, original),
        transform_pass=bool(
            finite and preparation_pass and all(parity.values()) and nx.passes(branch_error, 0.008)
            and nx.passes(residual_error, 0.008) and nx.passes(prep_error, 0.008) and nx.passes(scale_error, 0.008)
            and code_error <= 1
        ),
    )
    stages = dict(
        input_prepare=input_prepare,
        previous_projection=lambda: previous(aq, sa, fused),
        transition=lambda: transition(z, fused),
        next_projection=lambda: next_projection(q1, s1),
        online_activation_plus_gemm=lambda: core(*input_prepare()),
        offline_weight_prepare=offline_weights,
    )
    return (lambda: core(aq, sa)), check, expected, original, stages, meta


# ---- Single Q or K projection with RMSNorm + RoPE (qk_rope_experiment.py:13-294) ---------------


def validate_qk_config(c, backend, precision, distribution, tile):
    """Reject unsupported semantics before any device work (qk_rope_experiment.py:13-60)."""
    if backend not in ("qk-staged", "qk-fused") or precision != "int8":
        raise NotImplementedError("qk_rope supports qk-staged/qk-fused with INT8 only")
    if c.get("op") != "qk_rope":
        raise ValueError("operation must be qk_rope")
    for key in ("m", "n", "k"):
        if not _positive_int(c.get(key)):
            raise ValueError(f"{key} must be a positive integer")
    head_dim = c.get("head_dim", 128)
    if isinstance(head_dim, bool) or not isinstance(head_dim, Integral) or head_dim != 128 or c["n"] % 128:
        raise NotImplementedError("Q/K projection requires complete 128-wide heads")
    if c["k"] % 256:
        raise NotImplementedError("K must be divisible by H256; no implicit padding")
    if c["k"] > 131071:
        raise NotImplementedError("INT32 worst-case overflow bound exceeded")
    half = c.get("rope_half", 48)
    if isinstance(half, bool) or not isinstance(half, Integral) or not 1 <= half <= 64:
        raise ValueError("rope_half must be an integer in [1,64]")
    epsilon = c.get("epsilon", 1e-5)
    if isinstance(epsilon, bool) or not isinstance(epsilon, Real) or not np.isfinite(epsilon) or epsilon <= 0:
        raise ValueError("epsilon must be positive and finite")
    with np.errstate(over="ignore", under="ignore"):
        epsilon = np.float32(epsilon)
    if not np.isfinite(epsilon) or epsilon <= 0:
        raise ValueError("epsilon must remain positive and finite in FP32")
    if distribution not in DISTRIBUTIONS:
        raise ValueError("distribution must be normal, outliers or zeros")
    if not isinstance(tile, (tuple, list)) or len(tile) != 4:
        raise ValueError("tile must contain TM,TN,SIMD groups,M swizzle")
    if any(isinstance(v, bool) or not isinstance(v, Integral) for v in tile):
        raise ValueError("tile entries must be integers")
    tm, tn, groups, swizzle = tile
    if tm not in (16, 32, 64, 128) or tn not in (64, 128) or groups not in (4, 8):
        raise NotImplementedError("Q/K tile supports TM16/32/64/128, TN64/128, groups4/8")
    if swizzle <= 0:
        raise ValueError("tile swizzle must be positive")
    return dict(head_dim=128, rope_half=int(half), epsilon=float(epsilon), block_size=256)


def sample_complete_heads(n, head_dim=128, count=2):
    """Sampled head ids and every projection column of those heads."""
    if n <= 0 or head_dim <= 0 or n % head_dim or count <= 0:
        raise ValueError("sampling requires positive whole heads and positive count")
    heads = nx.sample_indices(n // head_dim, count)
    return heads, (heads[:, None] * head_dim + np.arange(head_dim)[None, :]).reshape(-1)


def prepare_qk_rope(c, backend, precision, seed, distribution, tile):
    cfg = validate_qk_config(c, backend, precision, distribution, tile)
    m, n, k = c["m"], c["n"], c["k"]
    dim, half, eps, block = (cfg[key] for key in ("head_dim", "rope_half", "epsilon", "block_size"))
    rng = np.random.default_rng(seed)
    x = _dev(rng.standard_normal((m, k), dtype=np.float32))
    w = _dev(rng.standard_normal((n, k), dtype=np.float32) * k**-0.5)
    if distribution == "zeros":
        x, w = torch.zeros_like(x), torch.zeros_like(w)
    elif distribution == "outliers":
        x, w = _outliers(x, 127), _outliers(w, 131)
    gamma = _dev(1 + 0.2 * rng.standard_normal(dim, dtype=np.float32))
    angles = rng.uniform(-np.pi, np.pi, size=(m, half)).astype(np.float32)
    cos, sin = _dev(np.cos(angles)), _dev(np.sin(angles))
    signs = torch.ones(k, dtype=torch.int8, device="cuda")
    rows = nx.sample_indices(m)
    heads, columns = sample_complete_heads(n, dim)

    def extract(output):
        # Head-major selection keeps each sampled head's complete D axis.
        return _f64(output.index_select(0, _idx(heads)).index_select(1, _idx(rows))).reshape(-1)

    def activation_prepare():
        # The online H + INT8 in one dispatch: the same codes and scales as the reference's
        # quantize(rotate(x)), whose two halves the stages below still time one by one.
        return rotate_quantize(x, block, signs)

    rotated_a, rotated_w = rotate(x, block, signs), rotate(w, block, signs)
    aq, sa = quantize(rotated_a, "int8", tag="qk_online")
    bq, sb = quantize(rotated_w, "int8", tag="qk_weight")

    def projection(q, scales):
        return gemm(q, bq, "int8", tile, a_scales=scales, b_scales=sb, output_dtype=BF)

    def postprocess(projected):
        return qk_norm_rope(projected, gamma, cos, sin, epsilon=eps, threads=tile[2] * 32)

    def staged(q, scales):
        return postprocess(projection(q, scales))

    def fused(q, scales):
        return projection_qk_rope(q, bq, gamma, cos, sin, "int8", tile, a_scales=scales, b_scales=sb, epsilon=eps)

    selected = fused if backend == "qk-fused" else staged
    projected = projection(aq, sa)
    staged_output = postprocess(projected)
    fused_output = fused(aq, sa)
    torch.cuda.synchronize()
    parity_error = nx.metrics(extract(fused_output), extract(staged_output))
    parity_exact = bool(torch.equal(fused_output, staged_output))
    ref_x, ref_w = _rows(x, rows), _rows(w, columns)
    ref_gamma, ref_cos, ref_sin = _f64(gamma), _rows(cos, rows), _rows(sin, rows)

    def reference(dot):
        return nx.qk_rope(dot.reshape(len(rows), len(heads), dim), ref_gamma, ref_cos, ref_sin,
                          epsilon=eps).reshape(-1)

    original_dot = ref_x @ ref_w.T
    original = reference(original_dot)
    decoded_a = _decoded(aq, sa, "int8", rows)
    decoded_w = _decoded(bq, sb, "int8", columns)
    decoded_dot = decoded_a @ decoded_w.T
    expected = reference(decoded_dot)
    ref_rotated_a, ref_rotated_w = nx.block_hadamard(ref_x, block), nx.block_hadamard(ref_w, block)
    ref_a_codes, ref_a_scales, ideal_a = nx.symmetric_int8(ref_rotated_a)
    ref_w_codes, ref_w_scales, ideal_w = nx.symmetric_int8(ref_rotated_w)
    rotation_a_error = nx.metrics(_rows(rotated_a, rows), ref_rotated_a)
    rotation_w_error = nx.metrics(_rows(rotated_w, columns), ref_rotated_w)
    a_scale_error = nx.metrics(_rows(sa[:, None], rows)[:, 0], ref_a_scales)
    w_scale_error = nx.metrics(_rows(sb[:, None], columns)[:, 0], ref_w_scales)
    a_code_diff = float(np.max(np.abs(_rows(aq, rows) - ref_a_codes)))
    w_code_diff = float(np.max(np.abs(_rows(bq, columns) - ref_w_codes)))
    a_prep_error, w_prep_error = nx.metrics(decoded_a, ideal_a), nx.metrics(decoded_w, ideal_w)
    dot_preservation = nx.metrics(ref_rotated_a @ ref_rotated_w.T, original_dot)
    sampled_projection = _grid(projected, rows, columns)
    projection_error = nx.metrics(sampled_projection, nx.bf16_round(decoded_dot))
    postprocess_error = nx.metrics(extract(staged_output), reference(sampled_projection))
    finite = all_finite((x, w, gamma, cos, sin, rotated_a, rotated_w, sa, sb, projected, staged_output, fused_output))
    positive_scales = bool((sa > 0).all().item() and (sb > 0).all().item())
    transform_pass = bool(
        finite and positive_scales and parity_exact
        and all(nx.passes(e, 1e-5) for e in (rotation_a_error, rotation_w_error, a_scale_error, w_scale_error))
        and nx.passes(dot_preservation, 1e-12)
        and all(nx.passes(e, 0.008) for e in (a_prep_error, w_prep_error, parity_error, projection_error,
                                              postprocess_error))
        and a_code_diff <= 1 and w_code_diff <= 1
    )
    meta = dict(
        online_activation_preparation="block Hadamard and INT8 in one dispatch (the codes and scales of quantize(rotate(x)))",
        compute_path=backend,
        operation_scope="one Q or K projection, not grouped QKV or attention",
        input_dtype="bf16",
        output_dtype="bf16",
        output_layout="head-major [H,M,128], contiguous",
        weight_layout="[H*128,K], ordinary single-projection order",
        reference="NumPy float64 dots with full K and every channel of sampled complete heads; explicit BF16 "
                  "projection/output",
        sample_rows=rows.tolist(),
        sample_heads=heads.tolist(),
        sample_cols=columns.tolist(),
        head_dim=dim,
        rope_half=half,
        epsilon=eps,
        projection_rounding="BF16 after FP32 INT8 dequantization, before RMS",
        normalization_rounding="none; FP32 RMS/gamma/RoPE before final BF16",
        rope_pairing="split-half (j,j+rope_half); remaining channels normalized but unrotated",
        rope_table_origin="synthetic independent random angles",
        gamma_sha256=hashlib.sha256(ref_gamma.astype(np.float32).tobytes()).hexdigest(),
        main_timing_scope="resident INT8 projection plus RMS/gamma/RoPE and head-major output",
        online_timing_scope="BF16 activation H256 + INT8 packing + projection + RMS/gamma/RoPE + head-major BF16 "
                            "output",
        weight_preparation_timed=True,
        weight_preparation_in_online=False,
        mac_operations=2 * m * n * k,
        all_preparation_values_finite=finite,
        positive_quantization_scales=positive_scales,
        paired_path_error=parity_error,
        paired_path_exact=parity_exact,
        paired_path_exact_required=True,
        projection_implementation_error=projection_error,
        postprocess_implementation_error=postprocess_error,
        activation_rotation_error=rotation_a_error,
        weight_rotation_error=rotation_w_error,
        activation_scale_error=a_scale_error,
        weight_scale_error=w_scale_error,
        activation_max_code_difference=a_code_diff,
        weight_max_code_difference=w_code_diff,
        activation_implementation_error=a_prep_error,
        weight_implementation_error=w_prep_error,
        ideal_activation_quantization_error=nx.metrics(ideal_a, ref_rotated_a),
        ideal_weight_quantization_error=nx.metrics(ideal_w, ref_rotated_w),
        ideal_decoded_quantization_error=nx.metrics(reference(ideal_a @ ideal_w.T), original),
        decoded_preparation_total_error=nx.metrics(expected, original),
        transform=dict(
            kind="normalized_block_sylvester_hadamard",
            block_size=block,
            sign_policy="all +1; same activation and weight transform",
            padding=0,
            float64_dot_preservation_error=dot_preservation,
        ),
        transform_pass=transform_pass,
    )
    stages = dict(
        activation_hadamard=lambda: rotate(x, block, signs),
        activation_quantization=lambda: quantize(rotated_a, "int8", tag="qk_online"),
        activation_prepare=activation_prepare,
        projection=lambda: projection(aq, sa),
        postprocess=lambda: postprocess(projected),
        online_activation_plus_gemm=lambda: selected(*activation_prepare()),
        offline_weight_prepare=lambda: quantize(rotate(w, block, signs), "int8", tag="qk_weight"),
    )
    return (lambda: selected(aq, sa)), extract, expected, original, stages, meta


def prepare_unsupported(c, backend, precision, seed, distribution, tile):
    raise NotImplementedError(
        f"{c['op']} is outside the quantized-projection path this library implements on MI355X")


PREPARE = {
    "gemm": prepare_gemm,
    "norm_hadamard_gemm": prepare_norm_hadamard_gemm,
    "gated_norm_hadamard_gemm": prepare_norm_hadamard_gemm,
    "rms_quant_gemm": prepare_rms_quant_gemm,
    "gate_epilogue_chain": prepare_gate_epilogue_chain,
    "qk_rope": prepare_qk_rope,
}
