"""The C ABI library on the host: it loads, exports every function
include/biv_hip.h declares, and reports errors as biv's backends do."""
import ctypes
import os
import re

import numpy as np
import pytest

from conftest import ROOT


def header_functions():
    text = open(os.path.join(ROOT, "include", "biv_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(biv_(?:hip|gguf)_\w+)\s*\(", text)))


def test_header_matches_python_binding():
    from biv_amd import hip
    assert header_functions() == sorted(hip.SYMBOLS)


def test_library_exports_every_symbol():
    from biv_amd import hip
    lib = hip.load()
    for name in header_functions():
        assert hasattr(lib, name), name


def test_numerics_without_device():
    from biv_amd import hip
    lib = hip.load()
    buf = ctypes.create_string_buffer(512)
    assert lib.biv_hip_numerics(None, buf, 512) == 0
    kv = dict(x.split("=", 1) for x in buf.value.decode().split(";"))
    assert kv["kind"] == "hip" and kv["arch"] == "gfx950" and kv["deterministic"] == "1"


def test_null_arguments_are_rejected():
    from biv_amd import hip
    lib = hip.load()
    assert lib.biv_hip_create(0, None) == -1
    assert lib.biv_hip_sync(None) == -1
    assert lib.biv_hip_moe_forward(None, None, None, 1, None, 0) == -1
    assert lib.biv_hip_device_bytes(None) == 0


def test_create_fails_loudly_without_gpu():
    """On a host with no gfx950 device, construction is an error (Error::Backend),
    never a silent CPU fallback."""
    from biv_amd import hip
    try:
        import torch
        if torch.cuda.is_available():
            pytest.skip("a GPU is present")
    except ImportError:
        pass
    with pytest.raises(hip.HipError) as e:
        hip.HipEngine(0)
    assert e.value.code == -3


def test_code_objects_are_gfx950():
    """The library carries gfx950 code objects (built by biv_amd.build)."""
    from biv_amd import hip
    data = open(hip.LIB_PATH, "rb").read()
    assert b"gfx950" in data


def test_cpp_host_mirror_compiles_and_throws_without_gpu(tmp_path):
    """include/biv_hip.hpp is standalone C++17 over the C ABI: g++ builds a
    program against libbiv_hip.so, and constructing an Engine on a host with
    no gfx950 device throws Error carrying BIV_HIP_E_DEVICE and the message
    (Error::Backend at construction)."""
    import subprocess
    src = tmp_path / "m.cpp"
    src.write_text(r'''
#include "biv_hip.hpp"
#include <cstdio>
int main() {
    try {
        biv::hip::Engine e(0);
        std::printf("constructed\n");
        return 2;
    } catch (const biv::hip::Error &err) {
        std::printf("code=%d msg=%s\n", err.code(), err.what());
        return err.code() == BIV_HIP_E_DEVICE ? 0 : 1;
    }
}
''')
    exe = tmp_path / "m"
    lib = os.path.join(ROOT, "biv_amd")
    subprocess.run(["g++", "-std=c++17", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), str(src), "-o",
                    str(exe), "-L", lib, "-lbiv_hip", f"-Wl,-rpath,{lib}"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "code=-3" in r.stdout and "device" in r.stdout
