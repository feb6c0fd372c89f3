"""The C-ABI library loads and exports every symbol include/moss_hip.h declares (CPU only)."""
import ctypes
import os
import re

from conftest import ROOT

from mosship import lib


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "moss_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(moss_hip_\w+)\s*\(", text)))


def test_header_declares_the_binding_list():
    assert declared_symbols() == sorted(lib.EXPORTED)


def test_library_exports_every_declared_symbol():
    L = lib.load()
    missing = [s for s in declared_symbols() if not hasattr(L, s)]
    assert not missing, missing
    assert L.moss_hip_abi_version() == 8


def test_capture_layout_matches_header():
    """The binding's capture offsets are the header's MOSS_HIP_CAP_* values, and the
    sections tile one step exactly."""
    text = open(os.path.join(ROOT, "include", "moss_hip.h")).read()
    vals = {m[0]: int(m[1]) for m in re.findall(r"\b(MOSS_HIP_CAP_\w+)\s*=\s*(\d+)", text)}
    assert vals["MOSS_HIP_CAP_STEP"] == lib.CAP_STEP
    assert (vals["MOSS_HIP_CAP_GLOBAL"], vals["MOSS_HIP_CAP_LOCAL"], vals["MOSS_HIP_CAP_PREFILL"]) == \
        (lib.CAP_GLOBAL, lib.CAP_LOCAL, lib.CAP_PREFILL)
    end = 0
    for name, (off, n) in sorted(lib.CAP.items(), key=lambda kv: kv[1][0]):
        assert vals["MOSS_HIP_CAP_" + name.upper()] == off
        assert off == end, name
        end = off + n
    assert end == lib.CAP_STEP


def test_error_paths_without_gpu():
    """Argument validation runs before any device call."""
    L = lib.load()
    h = ctypes.c_void_p()
    assert L.moss_hip_llm_create(None, 0, None, ctypes.byref(h)) == lib.EINVAL
    assert b"null" in L.moss_hip_last_error()
    assert L.moss_hip_llm_global_step(None, None) == lib.EINVAL
    assert L.moss_hip_llm_position(None) == -1
    assert L.moss_hip_codec_create(None, 0, None, ctypes.byref(h)) == lib.EINVAL
    assert L.moss_hip_codec_decode_chunk(None, None, 1, None) == lib.EINVAL
    assert L.moss_hip_codec_samples_per_frame(None) == -1
