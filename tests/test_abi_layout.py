"""The ctypes mirrors of the C ABI's argument structs (d2sd/_lib.py) against
include/d2sd.h: every field's offset and every struct's size, as a C compiler
lays them out (gcc on the header, no GPU)."""
import ctypes as C
import os
import re
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "d2-sd_amd"))

from d2sd import _lib  # noqa: E402

STRUCTS = {
    "PlanDesc": "d2sd_cascade_plan_desc",
    "PlanInfo": "d2sd_cascade_plan_info",
    "RunArgs": "d2sd_cascade_run_args",
    "KvAppendArgs": "d2sd_kv_append_args",
    "QkRopeArgs": "d2sd_qk_norm_rope_args",
    "TreeArgs": "d2sd_d3_tree_args",
    "AcceptArgs": "d2sd_greedy_accept_args",
    "SampleAcceptArgs": "d2sd_sample_accept_args",
}


def _c_layout():
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "d2sd.h"', "int main(void) {"]
    for py, c in STRUCTS.items():
        lines.append(f'  printf("{py} . %zu\\n", sizeof({c}));')
        for name, _ in getattr(_lib, py)._fields_:
            lines.append(f'  printf("{py} {name} %zu\\n", offsetof({c}, {name}));')
    lines += ["  return 0;", "}"]
    with tempfile.TemporaryDirectory() as tmp:
        src, exe = os.path.join(tmp, "layout.c"), os.path.join(tmp, "layout")
        Path(src).write_text("\n".join(lines) + "\n")
        subprocess.run([cc, "-std=c11", f"-I{ROOT / 'include'}", src, "-o", exe], check=True,
                       capture_output=True, text=True)
        out = subprocess.run([exe], check=True, capture_output=True, text=True).stdout
    layout = {}
    for line in out.splitlines():
        py, name, val = line.split()
        layout[(py, name)] = int(val)
    return layout


def _c_field_names(struct: str):
    """Member names of `typedef struct { ... } struct;` in include/d2sd.h, in
    declaration order (comments removed; `T a, b;` and `T* p;` forms)."""
    text = (ROOT / "include" / "d2sd.h").read_text()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = re.sub(r"//[^\n]*", " ", text)
    m = re.search(r"typedef struct\s*\{([^}]*)\}\s*" + struct + r"\s*;", text)
    assert m, struct
    names = []
    for decl in m.group(1).split(";"):
        decl = decl.strip()
        if not decl:
            continue
        parts = [p.strip() for p in decl.split(",")]
        names.append(re.findall(r"[A-Za-z_]\w*", parts[0])[-1])
        names += [re.findall(r"[A-Za-z_]\w*", p)[-1] for p in parts[1:]]
    return names


def test_ctypes_structs_name_every_c_field_in_order():
    for py, c in STRUCTS.items():
        assert [n for n, _ in getattr(_lib, py)._fields_] == _c_field_names(c), py


def test_ctypes_structs_match_the_c_header():
    layout = _c_layout()
    for py in STRUCTS:
        cls = getattr(_lib, py)
        assert C.sizeof(cls) == layout[(py, ".")], f"{py}: size {C.sizeof(cls)} != C {layout[(py, '.')]}"
        for name, _ in cls._fields_:
            off = getattr(cls, name).offset
            assert off == layout[(py, name)], f"{py}.{name}: offset {off} != C {layout[(py, name)]}"
