"""The C-ABI boundary, checked on the CPU: the library loads, exports every
entry point include/linattn_hip.h declares, and the ctypes structures match the
C layout (offsets printed by a probe compiled from the header)."""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from linattn_amd import _native as N

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "linattn_hip.h"

STRUCTS = {
    "la_kv": N.LaKV,
    "la_sparse_attn_args": N.LaSparseAttnArgs,
    "la_topk_args": N.LaTopkArgs,
    "la_quest_select_args": N.LaQuestSelectArgs,
    "la_indexer_args": N.LaIndexerArgs,
    "la_block_select_args": N.LaBlockSelectArgs,
    "la_prefill_args": N.LaPrefillArgs,
    "la_kv_append_args": N.LaKvAppendArgs,
    "la_gate_select_args": N.LaGateSelectArgs,
    "la_block_means_args": N.LaBlockMeansArgs,
    "la_xattn_select_args": N.LaXattnSelectArgs,
    "la_quest_decode_args": N.LaQuestDecodeArgs,
}


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(la_[a-z_0-9]+)\s*\(", text)))


def test_header_declares_the_exported_set():
    assert declared_functions() == sorted(N.EXPORTED)


def test_library_exports_every_declared_symbol():
    lib = N.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.la_abi_version() == N.ABI_VERSION
    assert isinstance(lib.la_last_error(), bytes)


def test_invalid_arguments_fail_without_a_gpu():
    """Argument validation runs before any HIP call, so it works on the CPU."""
    lib = N.load()
    a = N.LaSparseAttnArgs()
    kv = N.LaKV()
    assert lib.la_sparse_attention(ctypes.byref(a), ctypes.byref(kv), None) == N.LA_ERR_INVALID
    assert b"null" in lib.la_last_error()
    t = N.LaTopkArgs()
    assert lib.la_topk_rows(ctypes.byref(t), None) == N.LA_ERR_INVALID
    with pytest.raises(ValueError):
        N.check(N.LA_ERR_INVALID, "x")


def test_struct_layouts_match_the_header(tmp_path):
    lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void){"]
    for cname, py in STRUCTS.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in py._fields_:
            lines.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0;}")
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c99", "-o", str(exe), str(src)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    c = {}
    for line in out.splitlines():
        s, f, v = line.split()
        c[(s, f)] = int(v)
    for cname, py in STRUCTS.items():
        assert c[(cname, "size")] == ctypes.sizeof(py), cname
        for fname, _ in py._fields_:
            assert c[(cname, fname)] == getattr(py, fname).offset, (cname, fname)
