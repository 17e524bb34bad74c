"""Workload suites: the reference's versioned JSON schema (workloads.py:9-37).

A suite is ``{"schema_version": 1, "description": ..., "cases": [...]}``; each case has a
nonempty ``id``, an ``op`` and the positive integer shape fields of that op.  ``load`` takes a
path (so the reference's own ``workloads/*.json`` run unchanged) or the name of a suite shipped
in ``m5kernels_amd/harness/suites/``.
"""

from __future__ import annotations

import json
from pathlib import Path

SUITES = Path(__file__).resolve().parent / "suites"

FIELDS = {
    "gemm": ("m", "n", "k"),
    "norm_hadamard_gemm": ("m", "n", "k"),
    "gated_norm_hadamard_gemm": ("m", "n", "k"),
    "rms_quant_gemm": ("m", "n", "k"),
    "gate_epilogue_chain": ("m", "n", "k", "previous_k"),
    "qk_rope": ("m", "n", "k"),
    "attention": ("batch", "heads", "seq", "head_dim"),
    "rms_modulate": ("m", "n"),
    "swiglu": ("m", "n"),
}


def validate(c):
    """Return the case if its id and shape fields are valid; raise ValueError/KeyError else."""
    if not isinstance(c.get("id"), str) or not c["id"]:
        raise ValueError("nonempty id required")
    for f in FIELDS[c["op"]]:
        if type(c.get(f)) is not int or c[f] < 1:
            raise ValueError(f"{f} must be a positive integer")
    return c


# Widths of the H3 video/audio diffusion transformer (its public transformer config).
H3_CONFIG = dict(hidden_size=5376, num_attention_heads=56, attention_head_dim=128, ffn_dim=14336, text_dim=5120)


def load(name):
    """Suite document from a JSON path, a shipped suite name, "h3" or "h3-fused" (both generated
    from H3_CONFIG); case ids must be unique."""
    p = Path(name)
    if not p.exists():
        p = SUITES / f"{name}.json"
    if not p.exists() and name == "h3":
        data = dict(schema_version=1, description="H3 projection GEMMs and row ops at 128/1024/4096 tokens",
                    cases=h3_cases(H3_CONFIG))
    elif not p.exists() and name == "h3-fused":
        data = dict(schema_version=1, description="H3 fused activation-preparation projections at 128/4096/9914 tokens",
                    cases=h3_fused_cases(H3_CONFIG))
    else:
        data = json.loads(p.read_text())
    cases = [validate(c) for c in data["cases"]]
    if len({c["id"] for c in cases}) != len(cases):
        raise ValueError("duplicate case id")
    return data


def h3_cases(config, tokens=(128, 1024, 4096)):
    """GEMM shapes of the H3 transformer's projections (workloads.py:40-97) from its config
    dict (hidden_size, num_attention_heads, attention_head_dim, ffn_dim, text_dim), plus the
    per-token row ops; AdaLN-style projections are single-row (m = 1)."""
    h = config["hidden_size"]
    d = config["num_attention_heads"] * config["attention_head_dim"]
    f = config["ffn_dim"]
    projections = {
        "attn_q": (h, d), "attn_k": (h, d), "attn_v": (h, d), "attn_qkv_fused": (h, 3 * d),
        "attn_out": (d, h), "ffn_gate": (h, f), "ffn_up": (h, f), "ffn_gate_up_fused": (h, 2 * f),
        "ffn_down": (f, h), "text_in": (config["text_dim"], h), "video_in": (96, h), "audio_in": (32, h),
        "video_out": (h, 96), "audio_out": (h, 32),
    }
    cases = []
    for m in tokens:
        for name, (k, n) in projections.items():
            cases.append(dict(id=f"h3.{name}.m{m}", op="gemm", m=m, n=n, k=k, component=name,
                              shape_origin="official config; synthetic token count"))
        cases += [
            dict(id=f"h3.attention.s{m}", op="attention", batch=1, heads=config["num_attention_heads"], seq=m,
                 head_dim=config["attention_head_dim"], causal=False, component="dit_attention"),
            dict(id=f"h3.rms_modulate.m{m}", op="rms_modulate", m=m, n=h),
            dict(id=f"h3.swiglu.m{m}", op="swiglu", m=m, n=f),
        ]
    for name, k, n in [("adaln", h // 2, 18 * h), ("final_adaln", h // 2, 2 * h), ("time_in", 256, h),
                       ("time_out", h, h // 2)]:
        cases.append(dict(id=f"h3.{name}", op="gemm", m=1, k=k, n=n, component=name))
    return cases


def h3_fused_cases(config, tokens=(128, 4096, 9914)):
    """The fused projections of the H3 transformer at each token count, with the case ids and
    options of the reference's fused suites (workloads/h3-norm-hadamard.json,
    h3-gated-norm-hadamard.json, h3-shift-split.json, rms-quant.json, h3-gate-epilogue.json,
    h3-qk-rope.json): the norm + H256 + INT8 projections to Q and FFN-up, their residual-gated
    form, the FP32-rounding norm projection to Q (shift-split), the RMS-quantized Q projection
    (identity gamma, random gamma, random gamma with H256), the gate-epilogue chains
    attention -> FFN-up and FFN -> Q, and the Q/K projection with RoPE.  The shift-split and RMS
    cases are defined at 4096 and 9914 tokens only, as in the reference."""
    h = config["hidden_size"]
    d = config["num_attention_heads"] * config["attention_head_dim"]
    f = config["ffn_dim"]
    norm = dict(norm="rms", block_size=256, round_output="input")
    shift = dict(norm="rms", block_size=256, round_output="fp32", threads=256)
    rms = {"plain": (1, "identity"), "weighted": (1, "random"), "weighted_h256": (256, "random")}
    cases = []
    for m in tokens:
        for name, n in (("q", d), ("ffn_up", f)):
            cases.append(dict(id=f"h3.norm_{name}.m{m}", op="norm_hadamard_gemm", m=m, n=n, k=h, fusion=dict(norm)))
            cases.append(dict(id=f"h3.gated_{name}.m{m}", op="gated_norm_hadamard_gemm", m=m, n=n, k=h,
                              fusion=dict(norm)))
        if m != 128:
            cases.append(dict(id=f"h3.shift_q.m{m}", op="norm_hadamard_gemm", m=m, n=d, k=h, fusion=dict(shift)))
            for name, (block, gamma) in rms.items():
                cases.append(dict(id=f"rms.{name}.m{m}", op="rms_quant_gemm", m=m, n=d, k=h,
                                  rms_quant=dict(block_size=block, gamma=gamma, threads=256, epsilon=1e-5)))
        cases.append(dict(id=f"h3.chain_attention_to_ffn.m{m}", op="gate_epilogue_chain", m=m, k=h, n=f,
                          previous_k=d, previous_tile=[128, 64, 4, 8]))
        cases.append(dict(id=f"h3.chain_ffn_to_q.m{m}", op="gate_epilogue_chain", m=m, k=h, n=d, previous_k=f,
                          previous_tile=[128, 128, 8, 8]))
        cases.append(dict(id=f"h3.qk_rope.m{m}", op="qk_rope", m=m, k=h, n=d, head_dim=config["attention_head_dim"],
                          rope_half=48))
    return cases
