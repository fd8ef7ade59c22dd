"""Struct layouts of include/anneal_hip.h, as the C compiler lays them out, against the table a Go
binding of the header (its package init check) and the Python ctypes mirror (anneal_amd/_lib.py) assume.
CPU only: compiles an offsetof() probe of the header with gcc."""
import ctypes as C
import os
import subprocess

import pytest

from anneal_amd import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# (struct, field or None for sizeof) -> bytes: the Go binding's init() checks the same numbers
TABLE = {
    ("ah_buffer_desc", None): 40, ("ah_buffer_desc", "uop_idx"): 0, ("ah_buffer_desc", "size"): 8,
    ("ah_buffer_desc", "dtype"): 16, ("ah_buffer_desc", "slot"): 20, ("ah_buffer_desc", "rank"): 24,
    ("ah_buffer_desc", "shape"): 32,
    ("ah_exec_item", None): 64, ("ah_exec_item", "source"): 0, ("ah_exec_item", "bufs"): 8,
    ("ah_exec_item", "n_bufs"): 16, ("ah_exec_item", "sym_vars"): 24, ("ah_exec_item", "n_sym_vars"): 32,
    ("ah_exec_item", "local_size"): 36, ("ah_exec_item", "workgroup_count"): 48,
    ("ah_input", None): 24, ("ah_input", "uop_idx"): 0, ("ah_input", "data"): 8, ("ah_input", "n"): 16,
    ("ah_output", None): 24, ("ah_output", "data"): 8, ("ah_output", "n"): 16,
    ("ah_bench_result", None): 48, ("ah_bench_result", "min_us"): 0, ("ah_bench_result", "median_us"): 8,
    ("ah_bench_result", "max_us"): 16, ("ah_bench_result", "mean_us"): 24, ("ah_bench_result", "stddev_us"): 32,
    ("ah_bench_result", "cv"): 40,
}


@pytest.fixture(scope="module")
def c_layout(tmp_path_factory):
    d = tmp_path_factory.mktemp("layout")
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "anneal_hip.h"', "int main(void) {"]
    for (s, f), _ in TABLE.items():
        expr = f"sizeof({s})" if f is None else f"offsetof({s}, {f})"
        lines.append(f'    printf("%s %s %zu\\n", "{s}", "{f or "-"}", (size_t){expr});')
    lines.append("    return 0;\n}")
    src = d / "probe.c"
    src.write_text("\n".join(lines))
    exe = d / "probe"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    got = {}
    for line in out.splitlines():
        s, f, v = line.split()
        got[(s, None if f == "-" else f)] = int(v)
    return got


def test_c_header_matches_the_binding_table(c_layout):
    assert c_layout == TABLE


@pytest.mark.parametrize("cls,name", [(L.ah_buffer_desc, "ah_buffer_desc"), (L.ah_exec_item, "ah_exec_item"),
                                      (L.ah_input, "ah_input"), (L.ah_output, "ah_output"),
                                      (L.ah_bench_result, "ah_bench_result")])
def test_ctypes_mirror_matches_the_c_header(c_layout, cls, name):
    assert C.sizeof(cls) == c_layout[(name, None)]
    for (s, f), off in c_layout.items():
        if s == name and f is not None:
            assert getattr(cls, f).offset == off, f
