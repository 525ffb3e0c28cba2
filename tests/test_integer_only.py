"""The served path is integer-only, as the reference requires of a served artifact: "The served
artifact has no float or transcendental instruction" (/root/reference CHARTER.md:31, §3.6), and
its GPU evaluator is admitted only if the emitted module holds no floating-point, MMA or tensor
token (docs/labs/d11-exporter-float-trunk/instrument/build.rs:13-60 `admit_ptx`, which inspects
the emitted module, not the source spelling).

Two checks here, both on the CPU:
- the device sources under uor-r4_amd/csrc/ (comments removed) name no floating-point type and
  call no libm routine;
- the gfx950 code object inside the built library (this repository's own build, disassembled
  with the ROCm LLVM tools) holds no floating-point, transcendental or matrix opcode. This is the
  check that catches the compiler's own float sequences, e.g. its expansion of a 32-bit integer
  division through v_rcp_iflag_f32.
"""

import os
import re
import shutil
import struct
import subprocess

import pytest

from conftest import ROOT

CSRC = os.path.join(ROOT, "uor-r4_amd", "csrc")
LIB = os.path.join(ROOT, "uor-r4_amd", "lib", "libuor_fbs_hip.so")
LLVM = "/opt/rocm/llvm/bin"

# Device sources: the kernels and every header they include. fbs_api.cpp and the host test
# library are host code.
DEVICE_SOURCES = sorted(f for f in os.listdir(CSRC) if f.endswith((".hip", ".h")))

BANNED_TYPES = re.compile(r"\b(double|float|__half|__bf16|_Float16|bfloat16|__fp16)\b")
# libm and float intrinsics, as calls (a member or variable of the same name is not one).
BANNED_CALLS = re.compile(
    r"(?<![.\w>])(sqrtf?|rsqrtf?|cbrtf?|expf?|exp2f?|expm1f?|logf?|log2f?|log10f?|powf?|fmaf?|"
    r"floorf?|ceilf?|roundf?|truncf?|rintf?|ldexpf?|frexpf?|sinf?|cosf?|tanhf?|__fdividef|"
    r"__frcp_rn|__builtin_sqrt\w*|__builtin_amdgcn_rcp\w*|__builtin_amdgcn_rsq\w*|"
    r"__builtin_amdgcn_mfma\w*)\s*\(")
BANNED_INCLUDES = re.compile(r"#\s*include\s*<(cmath|math\.h|hip/hip_fp16\.h|hip/hip_bf16\.h)>")

# Opcode families of the emitted module that carry floating point or matrix arithmetic.
FLOAT_OPCODE = re.compile(
    r"^(v|s)_\w*(_f16|_f32|_f64|_bf16|f16_|f32_|f64_|bf16_|_fp8|_bf8)\w*$|"
    r"^v_(rcp|rsq|sqrt|exp|log|sin|cos|frac|ldexp|div_scale|div_fmas|div_fixup|fma|mac)\w*$|"
    r"^v_(mfma|smfmac|wmma|swmmac|dot)\w*$")


def strip_comments(text):
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def test_float_opcode_pattern_catches_the_known_families():
    for op in ("v_rcp_iflag_f32_e32", "v_cvt_f32_u32_e32", "v_cvt_u32_f32_e32", "v_mul_f32_e32",
               "v_sqrt_f64_e32", "v_rsq_f64_e32", "v_div_scale_f64", "v_fma_f64", "v_pk_fma_f32",
               "v_mfma_i32_16x16x64_i8", "v_dot4_i32_i8", "v_exp_f32_e32", "s_add_f32"):
        assert FLOAT_OPCODE.match(op), op
    for op in ("v_mad_u64_u32", "v_mul_hi_u32", "v_sad_u16", "v_add_co_u32_e32", "s_mul_i32",
               "v_lshlrev_b64", "v_cndmask_b32_e64", "ds_read_b128", "global_load_dwordx4",
               "v_ffbh_u32_e32", "v_alignbit_b32", "v_bfe_u32"):
        assert not FLOAT_OPCODE.match(op), op


@pytest.mark.parametrize("name", DEVICE_SOURCES)
def test_device_source_names_no_floating_point(name):
    text = open(os.path.join(CSRC, name)).read()
    assert not BANNED_INCLUDES.search(text), f"{name}: includes a floating-point header"
    code = strip_comments(text)
    hits = sorted({m.group(0) for m in BANNED_TYPES.finditer(code)} |
                  {m.group(1) for m in BANNED_CALLS.finditer(code)})
    assert not hits, f"{name}: floating point or libm in device code: {hits}"


def _disassemble(lib_path, workdir):
    """Disassembly of every gfx950 code object in the library. Its .hip_fatbin section holds one
    clang offload bundle per translation unit, back to back: the magic, an entry count, then per
    entry (offset from the bundle's start, size, target triple), all little-endian u64."""
    fat = os.path.join(workdir, "fatbin")
    subprocess.run(["objcopy", "--dump-section", f".hip_fatbin={fat}", lib_path,
                    os.path.join(workdir, "stripped.so")], check=True, capture_output=True)
    blob = open(fat, "rb").read()
    magic = b"__CLANG_OFFLOAD_BUNDLE__"
    starts = [m.start() for m in re.finditer(re.escape(magic), blob)]
    assert starts, "no offload bundle in the library"
    text = []
    for i, a in enumerate(starts):
        (entries,) = struct.unpack_from("<Q", blob, a + len(magic))
        at = a + len(magic) + 8
        for _ in range(entries):
            off, size, tlen = struct.unpack_from("<QQQ", blob, at)
            triple = blob[at + 24:at + 24 + tlen].decode()
            at += 24 + tlen
            if size and "gfx950" in triple:
                co = os.path.join(workdir, f"gfx950_{i}.co")
                open(co, "wb").write(blob[a + off:a + off + size])
                text.append(subprocess.run([os.path.join(LLVM, "llvm-objdump"), "-d", co],
                                           check=True, capture_output=True, text=True).stdout)
    return "\n".join(text)


@pytest.mark.skipif(not os.path.exists(LIB) or shutil.which("objcopy") is None
                    or not os.path.exists(os.path.join(LLVM, "llvm-objdump")),
                    reason="the built library or the ROCm LLVM tools are absent")
def test_emitted_gfx950_module_has_no_floating_point_opcode(tmp_path):
    dis = _disassemble(LIB, str(tmp_path))
    fn, kernels, bad = None, set(), {}
    for line in dis.splitlines():
        m = re.match(r"^[0-9a-f]+ <(.+)>:$", line)
        if m:
            fn = m.group(1)
            kernels.add(fn)
            continue
        m = re.match(r"^\s+([sv]_[a-z0-9_]+)\b", line)
        if m and FLOAT_OPCODE.match(m.group(1)):
            bad.setdefault(fn, set()).add(m.group(1))
    # Every kernel family of the library was read: decode, prefill, rows, the drawer index, the
    # discrete scorer and the copy read.
    for family in ("fbs_decode_pair", "fbs_prefill", "fbs_rows", "index_probe", "d11", "copy"):
        assert any(family in k for k in kernels), family
    assert not bad, f"floating-point opcodes in the emitted module: {bad}"
