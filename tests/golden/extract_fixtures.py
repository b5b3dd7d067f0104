"""Copies the MoE-path golden vectors out of the reference's own test fixtures.

Run once in a container where the reference is mounted:
    python tests/golden/extract_fixtures.py /root/reference

Only data is copied (inputs and expected outputs the reference's tests hold):
  * Tests/HydraFormatTests/Fixtures/mxfp4_{packed.bin,scales.bin,expected.f32}
    (written by the reference's tools/gen_mxfp4_fixture.py; used by MXFP4Tests.swift:19-47)
  * reference_ops.json keys "router", "swiglu", "rms_norm" (ReferenceOpsTests.swift)
  * reference_ops.json keys "sdpa_full", "sdpa_sliding"  (attention with sinks; written by the
    reference's tools/gen_reference_fixtures.py:100-128, 217-220)
  * gemma4_operators.json keys "gelu_tanh", "router", "rms_norm", "rms_norm_unscaled",
    "layer"                                              (Gemma4ReferenceTests.swift)
Nothing at test time reads the reference.
"""
import json
import os
import shutil
import sys

HERE = os.path.dirname(os.path.abspath(__file__))


def main(ref: str) -> None:
    fx = os.path.join(ref, "Tests/HydraFormatTests/Fixtures")
    for name in ["mxfp4_packed.bin", "mxfp4_scales.bin", "mxfp4_expected.f32"]:
        shutil.copyfile(os.path.join(fx, name), os.path.join(HERE, name))
    rfx = os.path.join(ref, "Tests/HydraReferenceTests/Fixtures")
    with open(os.path.join(rfx, "reference_ops.json")) as f:
        ops = json.load(f)
    with open(os.path.join(HERE, "reference_ops_moe.json"), "w") as f:
        json.dump({k: ops[k] for k in ["router", "swiglu", "rms_norm"]}, f)
    with open(os.path.join(HERE, "reference_ops_attention.json"), "w") as f:
        json.dump({k: ops[k] for k in ["sdpa_full", "sdpa_sliding"]}, f)
    with open(os.path.join(rfx, "gemma4_operators.json")) as f:
        gem = json.load(f)
    with open(os.path.join(HERE, "gemma4_moe.json"), "w") as f:
        json.dump({k: gem[k] for k in ["gelu_tanh", "router", "rms_norm", "rms_norm_unscaled",
                                       "layer"]}, f)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
