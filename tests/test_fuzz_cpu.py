"""Mutated models through the engine's model front end under AddressSanitizer
and UndefinedBehaviorSanitizer (host code only, built with g++).

The VapourSynth filter loads user-supplied model files and the ONNX Runtime EP
hands over serialized graphs, both decoded by the library's own protobuf reader
(onnx.cc), graph builder (graph.cc) and the EP's partition (ep.cc).
tests/fuzz_model_parse.cc truncates,
bit-flips, splices and pads valid models with oversized varints; every mutant
must be decoded or refused with an error. A sanitizer report (out-of-bounds
read, overflow, use of uninitialised memory) aborts the run and fails the test.
"""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

from arthip_amd import models

HERE = Path(__file__).resolve().parent
CSRC = HERE.parent / "arthip_amd" / "csrc"


@pytest.fixture(scope="module")
def fuzzer(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None or not Path("/opt/rocm/include/hip/hip_runtime.h").exists():
        pytest.skip("g++ or the HIP headers are not available")
    exe = tmp_path_factory.mktemp("fuzz") / "fuzz_model_parse"
    cmd = [gxx, "-std=c++17", "-O1", "-g", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
           "-I", str(CSRC), "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
           str(HERE / "fuzz_model_parse.cc"), str(CSRC / "onnx.cc"), str(CSRC / "graph.cc"),
           str(CSRC / "ep.cc"),
           "-o", str(exe)]
    subprocess.run(cmd, check=True, capture_output=True)
    return exe


@pytest.mark.parametrize("name,make,iters", [
    ("c4f32", lambda: models.c4f32().bytes(), 4000),
    ("r8f64", lambda: models.r8f64().bytes(), 300),
    ("shipped", lambda: (HERE / "golden" / "ArtCNN_R8F64_fp16.onnx").read_bytes(), 150),
    ("chroma_fp32", lambda: (HERE / "golden" / "ArtCNN_R8F64_Chroma.onnx").read_bytes(), 80),
])
def test_mutated_models_are_refused_cleanly(fuzzer, tmp_path, name, make, iters):
    model = tmp_path / f"{name}.onnx"
    model.write_bytes(make())
    r = subprocess.run([str(fuzzer), "7", str(iters), str(model)], capture_output=True,
                       text=True, timeout=600)
    assert r.returncode == 0, f"{name}: fuzzer failed\n{r.stdout[-2000:]}\n{r.stderr[-4000:]}"
    print(name, r.stdout.strip())
    # Some mutants still decode and build, so the later stages are reached too.
    counts = dict(zip(r.stdout.split()[0::2], map(int, r.stdout.split()[1::2])))
    assert counts["parsed"] > 0
