"""The host-pointer ABI's error policy without a GPU (CPU only): by default a compute call prints why and aborts
(there is no CPU path); in EIF_HIP_HOST_RECORD mode the call returns with its outputs untouched and the error is
readable once per thread. Each case runs in a child process. On a machine with a usable device the children
report that and the test skips."""
import os
import subprocess
import sys
import textwrap

import pytest

from conftest import ROOT

LIB = os.path.join(ROOT, "bitllm.c_amd", "libbitllm_hip.so")

CHILD = textwrap.dedent("""
    import ctypes as C, sys
    import numpy as np
    lib = C.CDLL(sys.argv[1])
    vp, i = C.c_void_p, C.c_int
    lib.eif_hip_host_last_error.argtypes = [vp, C.c_size_t]
    lib.eif_gpu_matmul_bitnet_f32.argtypes = [vp, vp, vp, vp, vp, vp, i, i]
    lib.eif_gpu_matmul_bitnet_f32.restype = C.c_bool
    lib.eif_matmul_bitnet_f32.argtypes = [vp, vp, vp, vp, vp, i, i]
    w = np.full((4, 16), 0x55, np.uint8)          # 4 rows x 64 columns of +1
    s = np.ones(4, np.float32); x = np.ones(64, np.float32)
    y = np.full(4, 7.0, np.float32)
    if lib.eif_gpu_matmul_bitnet_f32(None, w.ctypes.data, s.ctypes.data, x.ctypes.data, None, y.ctypes.data, 4, 64):
        print("DEVICE"); sys.exit(0)          # the seat ran on a device: nothing to check here
    if sys.argv[2] == "record":
        assert lib.eif_hip_set_host_error_mode(1) == 0
        assert lib.eif_hip_set_host_error_mode(7) == -1
    lib.eif_matmul_bitnet_f32(w.ctypes.data, s.ctypes.data, x.ctypes.data, None, y.ctypes.data, 4, 64)
    msg = C.create_string_buffer(256)
    code = lib.eif_hip_host_last_error(msg, 256)
    again = lib.eif_hip_host_last_error(None, 0)
    print("RETURNED", code, again, bool((y == 7.0).all()), msg.value.decode())
""")


def run(mode):
    assert os.path.exists(LIB), "libbitllm_hip.so not built"
    return subprocess.run([sys.executable, "-c", CHILD, LIB, mode], capture_output=True, text=True, timeout=120)


def test_default_mode_aborts_without_a_device():
    r = run("abort")
    if "DEVICE" in r.stdout:
        pytest.skip("a usable device is present")
    assert r.returncode != 0 and "RETURNED" not in r.stdout
    assert "eif_matmul_bitnet_f32" in r.stderr and "no CPU fallback" in r.stderr


def test_record_mode_returns_and_reports():
    r = run("record")
    if "DEVICE" in r.stdout:
        pytest.skip("a usable device is present")
    assert r.returncode == 0, r.stderr[-2000:]
    line = [l for l in r.stdout.splitlines() if l.startswith("RETURNED")][0].split(" ", 4)
    code, again, untouched, msg = int(line[1]), int(line[2]), line[3] == "True", line[4]
    assert code == -2 and again == 0 and untouched   # EIF_HIP_E_DEVICE, cleared by the first read
    assert msg.startswith("eif_matmul_bitnet_f32: ")
