"""The host-side model-file readers built with AddressSanitizer and UndefinedBehaviorSanitizer (g++, host code only:
svlm.cpp, gguf_model.cpp, gguf_ternary.cpp, qwen35_gguf.cpp, qwen35_file.cpp; the GPU side replaced by stand-ins in
tests/asan/harness.cpp) and fed seeded corruptions of SVLM, TTML, BitNet GGUF, Qwen3.5 GGUF and QWN5 files: no
sanitizer report, every call returns. CPU only; skipped without g++ or the HIP headers."""
import os
import shutil
import subprocess

import pytest

from conftest import ROOT
import synth
import model_files
from test_file_fuzz import mutations

SRC = os.path.join(ROOT, "bitllm.c_amd", "csrc")


@pytest.fixture(scope="module")
def harness(tmp_path_factory):
    if not shutil.which("g++") or not os.path.exists("/opt/rocm/include/hip/hip_runtime_api.h"):
        pytest.skip("g++ or the HIP headers absent")
    out = str(tmp_path_factory.mktemp("asan") / "harness")
    srcs = [os.path.join(ROOT, "tests", "asan", "harness.cpp")] + \
        [os.path.join(SRC, f) for f in ("gguf_model.cpp", "gguf_ternary.cpp", "qwen35_gguf.cpp", "qwen35_file.cpp",
                                        "svlm.cpp")]
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-omit-frame-pointer",
           "-D__HIP_PLATFORM_AMD__", "-I" + os.path.join(ROOT, "include"), "-I" + SRC, "-I/opt/rocm/include", *srcs,
           "-o", out, "-lpthread", "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return out


def run(harness, mode, files):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1", UBSAN_OPTIONS="halt_on_error=1")
    r = subprocess.run([harness, mode, *files], capture_output=True, text=True, env=env, timeout=600)
    assert r.returncode == 0 and "ERROR" not in r.stderr and "runtime error" not in r.stderr, r.stderr[-3000:]
    return r.stdout


def write_all(tmp_path, tag, base, seed, n, span):
    d = tmp_path / tag
    d.mkdir()
    files = []
    for i, b in enumerate(mutations(base, seed, n, span)):
        p = d / f"{i:04d}"
        p.write_bytes(b)
        files.append(str(p))
    return files


def test_readers_under_sanitizers(harness, tmp_path):
    from test_qwn5 import make
    cfg = synth.bitnet_config(128, 256, 1, 4, 2, 32, 64, 64, 32, 32, 0, 0, 0, rope_theta=10000.0)
    model_files.write_svlm(str(tmp_path / "b.svlm"), cfg, synth.bitnet_model((3, 32), cfg), 32)
    c2 = synth.bitnet_config(128, 256, 1, 4, 2, 32, 64, 64, 0, 0, 0, 0, 0, rope_theta=10000.0)
    model_files.write_ttml(str(tmp_path / "b.ttml"), c2, synth.bitnet_model((4, 32), c2), interleaved=1)
    svlm = write_all(tmp_path, "svlm", (tmp_path / "b.svlm").read_bytes(), 7, 400, 176) + \
        write_all(tmp_path, "ttml", (tmp_path / "b.ttml").read_bytes(), 8, 400, 84)
    gg, _ = model_files.bitnet_gguf(c2, (9,), proj_types=(model_files.GGUF_TL1, model_files.GGUF_F16, model_files.GGUF_Q4_0))
    q = model_files.qwen35_gguf((9,), dim=64, hidden=128, n_heads=2, n_kv_heads=1, head_dim=32, vocab=64, heads_k=2,
                          k_dim=16, v_dim=32, emb_type=model_files.GGUF_F16,
                          lin_types=(model_files.GGUF_Q8_0, model_files.GGUF_F16, model_files.GGUF_Q4_0))
    _, w, _ = make("tern_g32_hadamard")
    run(harness, "svlm", svlm + [str(tmp_path / "b.svlm"), str(tmp_path / "b.ttml")])
    run(harness, "bitnet", write_all(tmp_path, "gguf", gg, 9, 400, 2600))
    run(harness, "q35gguf", write_all(tmp_path, "q35", q, 10, 200, 12000))
    run(harness, "qwn5", write_all(tmp_path, "qwn5", w, 11, 400, 400))
