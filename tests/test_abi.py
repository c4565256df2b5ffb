"""The C-ABI libraries load and export every symbol include/*.h declares."""

import ctypes
import glob
import os
import re

from conftest import ROOT


def declared_symbols():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(sf_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_header_declares_entry_points():
    names = declared_symbols()
    for n in ("sf_cast_f32_bf16", "sf_cast_scatter_f32_bf16", "sf_pack_b16", "sf_unpack_b16",
              "sf_memcpy_async", "sf_host_alloc", "sf_cpu_adam_step", "sf_adam_update"):
        assert n in names


def test_libraries_export_every_declared_symbol():
    from test1_amd import _native

    hip = ctypes.CDLL(_native.HIP_LIB)
    cpu = ctypes.CDLL(_native.CPU_LIB)
    missing = [n for n in declared_symbols() if not (hasattr(hip, n) or hasattr(cpu, n))]
    assert not missing, f"declared but not exported: {missing}"
    # the Python bindings describe exactly the exported entry points
    assert set(_native.HIP_SIGNATURES) | set(_native.CPU_SIGNATURES) == declared_symbols()


def test_error_strings_and_version():
    from test1_amd import _native

    hip, cpu = _native.hip(), _native.cpu()
    assert hip.sf_abi_version() == cpu.sf_abi_version() == 3
    assert b"invalid" in hip.sf_error_string(9001)
    assert b"optimizer" in cpu.sf_error_string(9004)


def test_device_entry_points_reject_bad_arguments_without_a_gpu():
    # argument checks run on the host before any HIP call
    from test1_amd import _native

    hip = _native.hip()
    assert hip.sf_cast_f32_bf16(None, None, 10, None) == 9001
    assert hip.sf_cast_f32_bf16(None, None, 0, None) == 0
    assert hip.sf_memcpy_async(None, None, 16, 1, None) == 9001
    assert hip.sf_stage_f32_bf16(None, None, 10, None, 8, None) == 9001
    assert hip.sf_stage_f32_bf16(None, None, 0, None, 0, None) == 0
    assert hip.sf_copy_segs_b16(None, -1, 0, None) == 9001
    buf = (ctypes.c_uint16 * 64)()
    # overlapping cast source and destination
    assert hip.sf_cast_f32_bf16(ctypes.addressof(buf), ctypes.addressof(buf), 8, None) == 9005
    seg = (_native.SfSeg * 1)()
    seg[0].src, seg[0].dst, seg[0].n = 0, ctypes.addressof(buf), 8
    assert hip.sf_copy_segs_b16(seg, 1, 0, None) == 9001
