"""A C caller of include/kda_bt16_hip.h (CPU only).

The header compiles as C99 with every warning an error, a program built
from it links against libkda_bt16_hip.so, the struct layouts it sees
(sizeof, and offsetof of every field) are the ones the Python binding
(kda_bt16/_hip.py) passes, and the entry points that launch nothing answer
as the header documents: the ABI version, the error strings, the workspace
sizes and the argument checks that come before any device work.
"""

from __future__ import annotations

import ctypes
import shutil
import subprocess
from pathlib import Path

import pytest

from kda_bt16 import _hip

ROOT = Path(__file__).resolve().parents[1]
INCLUDE = ROOT / "include"
ROCM_LIB = "/opt/rocm/lib"

FWD_FIELDS = [f for f, _ in _hip.KdaBt16Args._fields_]
BWD_FIELDS = [f for f, _ in _hip.KdaBt16BwdArgs._fields_]

PROGRAM = r"""
#include <stddef.h>
#include <stdio.h>
#include "kda_bt16_hip.h"

#define OFF(T, f) printf("off %s %s %zu\n", #T, #f, offsetof(T, f))

int main(void) {
    KdaBt16Args a = {0};
    uint32_t count = 0;
    printf("size KdaBt16Args %zu\n", sizeof(KdaBt16Args));
    printf("size KdaBt16BwdArgs %zu\n", sizeof(KdaBt16BwdArgs));
@OFFSETS@
    printf("abi %d %d\n", kda_bt16_abi_version(), KDA_BT16_ABI_VERSION);
    printf("ws %zu\n", kda_bt16_workspace_bytes(1, 8192, 32, 128, 128));
    printf("rc fwd_null %d\n", kda_bt16_fwd_hip(NULL, NULL));
    printf("rc plan_null %d\n", kda_bt16_fwd_plan(NULL));
    printf("rc aborts_null %d\n", kda_bt16_fused_aborts(NULL, 0));
    printf("rc bwd_null %d\n", kda_bt16_bwd_hip(NULL, NULL));
    a.abi_version = KDA_BT16_ABI_VERSION + 1;
    printf("rc plan_abi %d\n", kda_bt16_fwd_plan(&a));
    a.abi_version = KDA_BT16_ABI_VERSION;
    a.B = 1; a.T = 16; a.H = 1; a.HV = 1; a.K = 64; a.V = 128;
    printf("rc plan_k64 %d\n", kda_bt16_fwd_plan(&a));
    printf("codes %d %d %d %d %d\n", KDA_BT16_OK, KDA_BT16_EINVAL, KDA_BT16_EUNSUPPORTED,
           KDA_BT16_EABI, KDA_BT16_ESCRATCH);
    printf("str %s\n", kda_bt16_strerror(KDA_BT16_EABI));
    (void)count;
    return 0;
}
"""


def _program() -> str:
    lines = [f"    OFF(KdaBt16Args, {f});" for f in FWD_FIELDS]
    lines += [f"    OFF(KdaBt16BwdArgs, {f});" for f in BWD_FIELDS]
    return PROGRAM.replace("@OFFSETS@", "\n".join(lines))


@pytest.fixture(scope="module")
def c_output(tmp_path_factory):
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    lib_dir = _hip.LIB_PATH.parent
    d = tmp_path_factory.mktemp("c_caller")
    src = d / "caller.c"
    src.write_text(_program())
    exe = d / "caller"
    cmd = [cc, "-std=c99", "-Wall", "-Wextra", "-Werror", "-pedantic", f"-I{INCLUDE}", str(src),
           "-o", str(exe), f"-L{lib_dir}", f"-l:{_hip.LIB_PATH.name}",
           f"-Wl,-rpath,{lib_dir}", f"-Wl,-rpath,{ROCM_LIB}", f"-Wl,-rpath-link,{ROCM_LIB}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    out = {}
    for line in r.stdout.splitlines():
        key, rest = line.split(" ", 1)
        out.setdefault(key, []).append(rest)
    return out


def test_struct_sizes_and_offsets_match_the_binding(c_output):
    sizes = dict(s.split() for s in c_output["size"])
    assert int(sizes["KdaBt16Args"]) == ctypes.sizeof(_hip.KdaBt16Args)
    assert int(sizes["KdaBt16BwdArgs"]) == ctypes.sizeof(_hip.KdaBt16BwdArgs)
    offs = {}
    for s in c_output["off"]:
        struct, field, off = s.split()
        offs[(struct, field)] = int(off)
    for f in FWD_FIELDS:
        assert offs[("KdaBt16Args", f)] == getattr(_hip.KdaBt16Args, f).offset, f
    for f in BWD_FIELDS:
        assert offs[("KdaBt16BwdArgs", f)] == getattr(_hip.KdaBt16BwdArgs, f).offset, f


def test_entry_points_without_launch(c_output):
    abi, macro = (int(x) for x in c_output["abi"][0].split())
    assert abi == macro == _hip.ABI_VERSION
    # one record of 17 KiB per (value head, chunk) at B=1 T=8192 HV=32
    assert int(c_output["ws"][0]) == 32 * 512 * 17408
    assert int(c_output["ws"][0]) == _hip.lib().kda_bt16_workspace_bytes(1, 8192, 32, 128, 128)
    rc = dict(s.split() for s in c_output["rc"])
    # the header's codes (as the C program sees them); the binding names ESCRATCH
    ok, einval, eunsup, eabi, escratch = (int(x) for x in c_output["codes"][0].split())
    assert ok == 0 and len({einval, eunsup, eabi, escratch}) == 4
    assert max(einval, eunsup, eabi, escratch) < 0
    assert escratch == _hip.ESCRATCH
    assert int(rc["fwd_null"]) == einval
    assert int(rc["plan_null"]) == einval
    assert int(rc["aborts_null"]) == einval
    assert int(rc["bwd_null"]) == einval
    assert int(rc["plan_abi"]) == eabi
    assert int(rc["plan_k64"]) == eunsup
    assert c_output["str"][0] == _hip.lib().kda_bt16_strerror(eabi).decode()
