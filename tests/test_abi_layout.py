"""Struct layouts across the bindings of include/vsplat.h.

A C program compiled against the header prints sizeof and offsetof of every
field of every struct the header declares; the test requires:

* the ctypes classes of vauss_amd/_lib.py to have exactly those fields, in
  that order, at those offsets, with that size (the Python binding);
* the Rust `#[repr(C)]` structs of the FFI stub in INTEGRATION.md to lay out
  identically under the C rules (the reference-side binding a maintainer
  would add);
* the oracle's camera, Adam and loss structs (oracle/vs_oracle.h, declared
  independently) to match the library's.
"""
import ctypes as C
import pathlib
import re
import shutil
import subprocess

import pytest

from vauss_amd import _lib

REPO = pathlib.Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "vsplat.h"

CTYPES = {
    "vs_camera": _lib.VsCamera, "vs_pose": _lib.VsPose, "vs_splats": _lib.VsSplats, "vs_fwd_out": _lib.VsFwdOut,
    "vs_grads": _lib.VsGrads, "vs_stage_times": _lib.VsStageTimes, "vs_state_view": _lib.VsStateView,
    "vs_loss_cfg": _lib.VsLossCfg, "vs_adam_step": _lib.VsAdamStep, "vs_update_out": _lib.VsUpdateOut,
    "vs_sh_step_params": _lib.VsShStepParams,
}
ORACLE_TWINS = {"or_camera": "vs_camera", "or_adam": "vs_adam_step", "or_loss_cfg": "vs_loss_cfg"}


def _header_structs():
    """struct name -> field names, from the header text."""
    text = HEADER.read_text()
    out = {}
    for m in re.finditer(r"typedef struct (vs_\w+) \{(.*?)\} \1;", text, re.S):
        body = re.sub(r"/\*.*?\*/", "", m.group(2), flags=re.S)
        fields = []
        for decl in body.split(";"):
            decl = decl.strip()
            if not decl:
                continue
            # "float fx, fy, cx, cy" or "const float* transforms" or "float kb4[4]"
            names = decl.split(",")
            first = re.match(r"(.*?)([A-Za-z_]\w*)\s*(\[\d+\])?$", names[0].strip())
            fields.append(first.group(2))
            for extra in names[1:]:
                fields.append(re.match(r"\s*\**\s*([A-Za-z_]\w*)", extra).group(1))
        out[m.group(1)] = fields
    return out


def _c_layout(tmp_path, structs, extra_include=None):
    """{struct: (size, {field: offset})} as the C compiler lays them out."""
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    lines = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"']
    if extra_include:
        lines.append(f'#include "{extra_include}"')
    lines.append("int main(void) {")
    for name, fields in structs.items():
        lines.append(f'  printf("S {name} %zu\\n", sizeof({name}));')
        for f in fields:
            lines.append(f'  printf("F {name} {f} %zu\\n", offsetof({name}, {f}));')
    lines += ["  return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run([cc, "-std=c11", "-Wall", "-Werror", "-o", str(exe), str(src)], check=True)
    out = {}
    for line in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.splitlines():
        kind, name, *rest = line.split()
        if kind == "S":
            out.setdefault(name, [0, {}])[0] = int(rest[0])
        else:
            out.setdefault(name, [0, {}])[1][rest[0]] = int(rest[1])
    return out


def test_header_structs_all_bound():
    assert set(_header_structs()) == set(CTYPES)


def test_ctypes_layouts_match_the_header(tmp_path):
    structs = _header_structs()
    lay = _c_layout(tmp_path, structs)
    for name, cls in CTYPES.items():
        size, offs = lay[name]
        assert [f[0] for f in cls._fields_] == structs[name], name
        assert C.sizeof(cls) == size, name
        for f, _ in cls._fields_:
            assert getattr(cls, f).offset == offs[f], (name, f)


def test_oracle_structs_match_the_library(tmp_path):
    oracle_h = REPO / "oracle" / "vs_oracle.h"
    text = oracle_h.read_text()
    structs = {}
    for m in re.finditer(r"typedef struct (or_\w+) \{(.*?)\} \1;", text, re.S):
        if m.group(1) in ORACLE_TWINS:
            structs[m.group(1)] = None
    lib = _header_structs()
    for o, v in ORACLE_TWINS.items():
        structs[o] = lib[v]
    lay = _c_layout(tmp_path, structs, extra_include=oracle_h)
    ref = _c_layout(tmp_path / "..", {v: lib[v] for v in ORACLE_TWINS.values()})
    for o, v in ORACLE_TWINS.items():
        assert lay[o] == ref[v], (o, v)


# ---- the documented Rust binding --------------------------------------------------

_RUST_SIZES = {"i32": 4, "u32": 4, "f32": 4, "f64": 8, "u64": 8, "i64": 8, "u16": 2, "u8": 1, "c_int": 4}


def _rust_structs():
    doc = (REPO / "INTEGRATION.md").read_text()
    blocks = re.findall(r"```rust\n(.*?)```", doc, re.S)
    out = {}
    for block in blocks:
        block = re.sub(r"/\*.*?\*/", "", block, flags=re.S)
        block = re.sub(r"//[^\n]*", "", block)
        for m in re.finditer(r"pub struct (vs_\w+) \{(.*?)\}", block, re.S):
            fields = []
            for decl in m.group(2).split(","):
                decl = decl.strip()
                if not decl:
                    continue
                fm = re.match(r"pub (\w+)\s*:\s*(.+)$", decl, re.S)
                if fm is None:          # an opaque handle (`_p: [u8; 0]`)
                    fields = None
                    break
                fields.append((fm.group(1), " ".join(fm.group(2).split())))
            if fields is not None:
                out[m.group(1)] = fields
    return out


def _rust_size_align(ty):
    arr = re.match(r"\[(.+);\s*(\d+)\]$", ty)
    if arr:
        s, a = _rust_size_align(arr.group(1).strip())
        return s * int(arr.group(2)), a
    if ty.startswith("*const") or ty.startswith("*mut"):
        return 8, 8
    s = _RUST_SIZES[ty]
    return s, s


def test_rust_binding_matches_the_header(tmp_path):
    rust = _rust_structs()
    structs = _header_structs()
    lay = _c_layout(tmp_path, structs)
    documented = set(rust)
    assert {"vs_camera", "vs_pose", "vs_splats", "vs_fwd_out", "vs_grads", "vs_adam_step", "vs_update_out",
            "vs_sh_step_params", "vs_loss_cfg"} <= documented
    for name in documented:
        fields = rust[name]
        assert [f for f, _ in fields] == structs[name], name
        off, align = 0, 1
        size, offs = lay[name]
        for f, ty in fields:
            s, a = _rust_size_align(ty)
            off = (off + a - 1) // a * a
            assert off == offs[f], (name, f, off, offs[f])
            off += s
            align = max(align, a)
        assert (off + align - 1) // align * align == size, name


def _header_functions():
    """function name -> parameter count, from the header's declarations."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"^[A-Za-z_][\w\s\*]*?\b(vs_\w+)\s*\(([^;{]*?)\)\s*;", text, re.M | re.S):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_rust_binding_declares_every_entry_point():
    doc = (REPO / "INTEGRATION.md").read_text()
    block = re.search(r"```rust\n// crates/splat-train-hip/src/ffi.rs\n(.*?)```", doc, re.S).group(1)
    block = re.search(r'extern "C" \{(.*?)\n\}', block, re.S).group(1)
    rust = {}
    for m in re.finditer(r"pub fn (vs_\w+)\(([^()]*)\)\s*(?:->[^;]+)?;", block, re.S):
        params = m.group(2).strip()
        rust[m.group(1)] = 0 if not params else params.count(",") + 1 - params.rstrip().endswith(",")
    header = _header_functions()
    assert len(header) >= 36 and set(header) == set(_lib.SIGNATURES)
    assert set(rust) == set(header), (set(header) - set(rust), set(rust) - set(header))
    for name, n in header.items():
        assert rust[name] == n, (name, rust[name], n)


def test_header_constants_match_the_bindings():
    """The state view's projected-row stride, which a binding has to repeat."""
    text = HEADER.read_text()
    stride = int(re.search(r"#define VS_PROJ_ROW_FLOATS (\d+)u", text).group(1))
    assert stride == _lib.PROJ_ROW_FLOATS == 16
