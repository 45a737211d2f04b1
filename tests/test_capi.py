"""The C ABI without a GPU: the library loads, exports every function that
include/logkv_hip.h declares, the ctypes table covers exactly those, and every
ctypes struct has the header's layout (offsets and sizes from a gcc-compiled
probe of the header)."""

import ctypes as C
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from logkv_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "logkv_hip.h"


def header_text():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def declared_functions():
    return set(re.findall(r"\b(logkv_[a-z0-9_]+)\s*\(", header_text()))


def declared_structs():
    out = {}
    for body, name in re.findall(r"typedef struct \w+ \{(.*?)\} (\w+);", header_text(), flags=re.S):
        fields = []
        for decl in body.split(";"):
            decl = decl.strip()
            if not decl:
                continue
            names = decl.split(None, 1)[1] if not decl.startswith("const") else decl.split(None, 2)[2]
            for n in names.split(","):
                fields.append(n.strip().lstrip("*").strip())
        out[name] = fields
    return out


def test_library_exports_every_declared_function():
    if not _lib.LIB_PATH.exists():
        pytest.skip("liblogkv_hip.so is not built")
    handle = C.CDLL(str(_lib.LIB_PATH))
    names = declared_functions()
    assert names, "no declarations parsed"
    for name in sorted(names):
        assert hasattr(handle, name), name
    assert names == set(_lib.SIGNATURES), names ^ set(_lib.SIGNATURES)


STRUCTS = {
    "logkv_ladder_view": _lib.LadderView, "logkv_rows_view": _lib.RowsView,
    "logkv_route_params": _lib.RouteParams, "logkv_span_args": _lib.SpanArgs,
    "logkv_partition_args": _lib.PartitionArgs, "logkv_readout_view": _lib.ReadoutView,
    "logkv_pack_args": _lib.PackArgs, "logkv_attention_args": _lib.AttentionArgs,
    "logkv_alpha_select_args": _lib.AlphaSelectArgs, "logkv_op_log_view": _lib.OpLogView,
    "logkv_beta_args": _lib.BetaArgs, "logkv_slot_pack_args": _lib.SlotPackArgs,
    "logkv_attention_grad_args": _lib.AttentionGradArgs, "logkv_recent_args": _lib.RecentArgs,
}


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc")
def test_ctypes_structs_match_header_layout(tmp_path):
    structs = declared_structs()
    assert set(structs) == set(STRUCTS)
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void) {"]
    for name, fields in structs.items():
        lines.append(f'  printf("{name} sizeof %zu\\n", sizeof({name}));')
        for f in fields:
            lines.append(f'  printf("{name} {f} %zu\\n", offsetof({name}, {f}));')
    lines.append("  return 0;\n}")
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", str(src), "-o", str(exe)], check=True)
    layout = {}
    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        s, f, v = line.split()
        layout[(s, f)] = int(v)
    for name, cls in STRUCTS.items():
        assert C.sizeof(cls) == layout[(name, "sizeof")], name
        c_fields = [f for f, _ in cls._fields_]
        assert c_fields == structs[name], name
        for f in c_fields:
            assert getattr(cls, f).offset == layout[(name, f)], (name, f)
