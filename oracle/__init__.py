"""CPU oracle for the AnimaXS attention + quantized-linear hot path.

TEST INFRASTRUCTURE ONLY.  This package restates the reference algorithms on
the CPU (numpy for byte/integer arithmetic, torch-CPU fp32 for floating point)
so the HIP library can be checked against them.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only to compare against: the product library (``animaxs_amd``)
never imports, links or calls anything here, and has no CPU fallback.

Every function cites the reference file:line it follows (paths relative to the
reference repository root).  How each function is pinned (golden vectors,
known answers, closed forms, brute force) is listed in ``PINNING`` below and
exercised by ``tests/test_oracle_*.py``.
"""

from . import quant, rope, norms, attention, inputs, blocks, dit_io, probe  # noqa: F401

# function -> the independent checks that pin it (see tests/test_oracle_*.py)
PINNING = {
    "quant.dequant_w4 / dequant_w4_matrix": (
        "known answers of AnimaXSTests/QuantDecoderTests.swift:23-60 and "
        "MetalExecutionTests.swift:28-65,170-257; row reset at K=68; "
        "bit patterns compared with an independent per-element fp64 decode"),
    "quant.dequant_w8 / dequant_w8_matrix": (
        "QuantDecoderTests.swift:64-93; fp16-subnormal scale/zero bit patterns of "
        "MetalExecutionTests.swift:115-168; row reset at K=65"),
    "quant.dequant_to_half": (
        "MetalExecutionTests.swift:28-65 (0x6E,0.5,-0.25 -> 6.75, 2.75) and the "
        "row-aware RNE16 bit patterns of :170-257; exhaustive check against "
        "fp64 arithmetic followed by numpy's RNE cast"),
    "rope.dit_rope_table": (
        "golden table scripts/oracle_out/dit_rope_oracle.npz (32x32 grid, "
        "fixture tests/golden/dit_rope_subset.npz); anchors of "
        "DitRoPETests.swift:24-88; grid-size invariance (token h*W+w)"),
    "rope.neox_rope_table": (
        "closed form cos/sin(pos * theta^(-2j/128)) checked in fp64; "
        "QwenNumerics.ropeNeoX equivalence (rotate-half form) on random input"),
    "rope.apply_split_half": (
        "DiTBlockTests.swift:18-63 hand values (90/180 degree rotations, "
        "split-half vs adjacent pairing)"),
    "norms.rms_norm / rms_norm_heads": (
        "DiTBlockTests.swift:92-114 closed form; torch.nn.functional.rms_norm"),
    "norms.layer_norm_modulated": (
        "DiTBlockTests.swift:66-88 hand values; torch.nn.functional.layer_norm"),
    "norms.gelu_erf": "DiTBlockTests.swift:168-172 values; math.erf in fp64",
    "attention.sdpa": (
        "fp64 brute force on small shapes; zero-Q/K mean-of-V special case "
        "(AttentionExecutorTests.swift:460-504); last-V-row (c+1)/512 case "
        "(:64-88); GQA 0,0,1,1 (:90-111, GqaHeadMappingTests.swift:23-89); "
        "tiny 2x3 case (DiTBlockTests.swift:117-147); additive finfo.min/4 mask "
        "equivalence (scripts/qwen_comfy_oracle.py:233-248)"),
    "dit_io.timestep_sinusoid": (
        "known answers of AnimaXSTests/TimestepEmbedderTests.swift:18-34 (cos/sin first 8 "
        "at sigma 1) and DiTInputTests.swift:67-73; fp64 closed form at every schedule sigma"),
    "dit_io.patchify17 / unpatchify16 / unpatchify_velocity16": (
        "markers of DiTInputTests.swift:14-52; hand-computed entries of the 4x6 input of "
        "MetalExecutionTests.swift:548-592; round trip; equality with the reshape/permute "
        "form of scripts/dit_source_oracle.py:367-382"),
    "dit_io.euler_step / flow_to_denoised": (
        "hand-computed values of the MetalExecutionTests.swift:680-710 vectors; next_sigma = 0 "
        "returns denoised; flow then Euler equals x + dsigma * velocity"),
    "dit_io.prepare / final_layer": (
        "closed forms with identity projections (emb = raw / sqrt(0.5 + eps), "
        "adaln = SiLU(raw)); final layer on alternating-sign rows with exact fp16 "
        "shift/scale outputs (detects a shift/scale swap and layout errors)"),
    "blocks.dit_block": (
        "composition of pinned parts following scripts/dit_block0_oracle.py:327-391; "
        "zero-gate identity and zero-weight invariants; closed-form blocks against fp64 brute "
        "force (Q = K = 0 with identity V/O/MLP projections; a 2x2 grid where only RoPE and the "
        "distinct self Q/K norm weights shape the softmax; a cross branch with non-zero Q/K and "
        "distinct cross norm weights) that reject swapped shift/scale, another branch's gate, "
        "cross K/V from x, a missing Q or K RoPE, a Q or K normalised with the other's weight, "
        "a dropped cross Q or K norm, the self weights in the cross branch and RoPE on cross Q/K"),
    "probe.probe_stats / accumulate": (
        "known answers of AnimaXSTests/NumericalMonitorTests.swift:83-123 (float_to_half_probe "
        "input: every flag, first index 2, max 70000) and :167-189 (fp16 NaN/+Inf first index 1; "
        "fp32 -Inf and 80000 overflow, max 80000); closed forms (all finite: no flag, max of |v|; "
        "65504 is not an overflow, its successor is; -0.0 counts as 0; an offender at index k "
        "is first)"),
    "blocks.qwen_layer": (
        "composition following QwenEncoderMetal.swift:244-303 and "
        "scripts/qwen_comfy_oracle.py:268-300; zero-projection, causality, padding and "
        "sequence-independence invariants; a closed-form layer with W8 identity/doubling codes "
        "(129 -> 1, 130 -> 2) against fp64 brute force that rejects a dropped Q or K norm, one "
        "side using the other's norm weight, RoPE missing on Q or K, a missing causal mask, the "
        "input-norm weight in the post-attention norm and gate/up swapped in the SwiGLU"),
}
