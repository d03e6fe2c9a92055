"""The drop-in boundary: libh3_gpu_hip.so loads, exports every entry point
declared in include/h3_gpu.h and include/h3_hip.h with C linkage, fails
cleanly without a device, and -- where the reference tree is present -- the
reference engine's own DiT model layer (h3_dit.c, h3_dit_schedule.c,
h3_weights.c, h3_safetensors.c, h3_host.c) compiles against include/h3_gpu.h
and links against this library with no unresolved device symbol.  CPU only:
no compute call is made."""
import ctypes as C
import os
import re
import subprocess
import tempfile

import pytest

import h3hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("h3_gpu.h", "h3_hip.h")]
REFERENCE = "/root/reference"


def declared_functions(path):
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b(h3_(?:gpu|hip)_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def exported_symbols():
    out = subprocess.run(["nm", "-D", "--defined-only", h3hip.LIB_PATH],
                         capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_every_declared_entry_point_is_exported():
    exported = exported_symbols()
    names = [n for h in HEADERS for n in declared_functions(h)]
    assert len(names) > 100
    missing = [n for n in names if n not in exported]
    assert not missing, missing


def test_reference_api_surface_is_complete():
    """Every function the reference header declares is declared here too,
    with the same name (the signatures are compiled against in the link
    test below)."""
    if not os.path.isdir(REFERENCE):
        pytest.skip("reference tree not present")
    ref = declared_functions(os.path.join(REFERENCE, "h3_gpu.h"))
    ours = set(declared_functions(HEADERS[0]))
    assert [n for n in ref if n not in ours] == []


def test_library_loads_and_host_entry_points_work():
    L = h3hip.lib()
    assert L.h3_gpu_error(None) == b"unknown HIP error"
    assert L.h3_gpu_tensor_elements(None) == 0
    assert L.h3_gpu_begin(None) == 0 and L.h3_gpu_submit(None) == 0


def test_create_fails_cleanly_without_a_device():
    L = h3hip.lib()
    count = C.c_int(0)
    hip = C.CDLL("libamdhip64.so")
    if hip.hipGetDeviceCount(C.byref(count)) == 0 and count.value > 0:
        pytest.skip("a device is present")
    err = C.create_string_buffer(256)
    assert not L.h3_gpu_create(None, err, 256)
    assert b"no HIP device" in err.value


def test_reference_model_layer_links_against_this_backend():
    """The reference's C model layer, compiled from its sources where they lie
    (nothing is copied) with this repository's include/h3_gpu.h first on the
    include path, links into a shared object with -lh3_gpu_hip and leaves no
    h3_gpu_* symbol undefined."""
    if not os.path.isdir(REFERENCE):
        pytest.skip("reference tree not present")
    units = ["h3_dit.c", "h3_dit_schedule.c", "h3_weights.c",
             "h3_safetensors.c", "h3_host.c"]
    with tempfile.TemporaryDirectory() as tmp:
        objs = []
        for u in units:
            obj = os.path.join(tmp, u + ".o")
            subprocess.run(["gcc", "-std=c11", "-O1", "-fPIC", "-D_GNU_SOURCE",
                            "-I", os.path.join(ROOT, "include"), "-I",
                            REFERENCE, "-c", os.path.join(REFERENCE, u), "-o",
                            obj], check=True, capture_output=True)
            objs.append(obj)
        so = os.path.join(tmp, "libdit.so")
        lib_dir = os.path.dirname(h3hip.LIB_PATH)
        subprocess.run(["gcc", "-shared", "-o", so] + objs +
                       ["-L", lib_dir, "-lh3_gpu_hip", "-lm", "-lpthread",
                        "-Wl,--no-undefined", "-Wl,-rpath," + lib_dir],
                       check=True, capture_output=True)
        undef = subprocess.run(["nm", "-D", "--undefined-only", so],
                               capture_output=True, text=True).stdout
        assert not re.search(r"\bh3_gpu_", "\n".join(
            l for l in undef.splitlines() if "h3_gpu" in l and " U " in l
            and l.split()[-1] not in exported_symbols()))
