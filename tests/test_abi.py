"""C-ABI contract checks that need no GPU: the library loads, exports every
function include/*.h declares, and device-less initialisation fails with
LT_ERR_DEVICE (the reference's failed GpuContext.init -> CPU fallback,
main.zig:1889-1892)."""
import ctypes as C
import glob
import os
import re
import subprocess
import sys

import pytest

import llmtoy_amd as lt
from llmtoy_amd import lib as ltlib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(lt_[a-z0-9_]+)\s*\(", text))
    return names


def test_header_declares_the_binding_surface():
    assert declared_symbols() == set(ltlib.EXPORTS)


def test_library_exports_every_declared_symbol():
    L = lt.load_library()
    for name in declared_symbols():
        assert hasattr(L, name), name


def test_library_is_gfx950_code_object():
    # the offload bundle inside the .so names the target it was built for
    data = open(ltlib.LIB_PATH, "rb").read()
    assert b"gfx950" in data


def test_force_no_device_reports_device_error():
    code = ("import sys; sys.path.insert(0, %r)\n"
            "import llmtoy_amd as lt\n"
            "try:\n    lt.Context(0)\nexcept lt.lib.DeviceError as e:\n    print('DEVICE', e.code)\n") % (
                os.path.join(ROOT, "llmtoy-zig_amd"))
    env = dict(os.environ, LT_FORCE_NO_DEVICE="1")
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=120)
    assert "DEVICE 3" in out.stdout, out.stdout + out.stderr


CPP_TEST = os.path.join(ROOT, "tests", "cpp", "build", "test_host_ops")


def test_cpp_host_layer_builds_and_lists_tests():
    # the C++ mirror of the reference op API (llmtoy-zig_amd/host/llmtoy_ops.hpp)
    out = subprocess.run([CPP_TEST, "--list"], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0
    names = out.stdout.splitlines()
    assert "gpu matvec Q4_K scale" in names and len(names) == 12


@pytest.mark.gpu
def test_gpu_cpp_host_layer_parity():
    print("running tests/cpp/build/test_host_ops", flush=True)
    out = subprocess.run([CPP_TEST], capture_output=True, text=True, timeout=120)
    print(out.stdout[-3000:])
    assert out.returncode == 0 and "ALL PASSED" in out.stdout, out.stdout + out.stderr


def test_null_arguments_are_invalid_without_touching_a_device():
    L = lt.load_library()
    assert L.lt_init(0, None) == ltlib.LT_ERR_INVALID
    assert L.lt_sync(None) == ltlib.LT_ERR_INVALID
    assert L.lt_tensor_bytes(None) == 0
    assert L.lt_last_error(None) == b"null context"
