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
    assert L.moss_hip_abi_version() == 6


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
