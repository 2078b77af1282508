"""CPU: the Zig drop-in files (zig/attention_hip.zig, zig/hip_context.zig) bind exactly the C-ABI that
include/llmgen_attn.h declares and the library exports.

No Zig toolchain exists in this image, so the files are checked mechanically: every `extern fn` is parsed and its
name, argument count, argument types (in order) and return type are compared with the C declaration of the same
name, under the C <-> Zig type correspondence of the reference's own bindings (attention_v1.zig:10-48,
cuda_context.zig:1-11, memory.zig:1-11).  The execute body is checked for the calls the engine's operator makes.
"""
from __future__ import annotations

import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ZIG = os.path.join(ROOT, "zig")
HEADER = os.path.join(ROOT, "include", "llmgen_attn.h")


def _strip_c_comments(s: str) -> str:
    s = re.sub(r"/\*.*?\*/", " ", s, flags=re.S)
    return re.sub(r"//[^\n]*", " ", s)


def _c_type(t: str) -> str:
    t = " ".join(t.replace("*", " * ").split())
    t = re.sub(r"\s*\*", "*", t).strip()
    table = {
        "int": "int", "float": "f32", "size_t": "usize", "void": "void",
        "size_t*": "*usize", "int*": "*int", "char*": "[*c]u8",
    }
    if t in table:
        return table[t]
    if t.endswith("*"):
        return "cptr" if t.startswith("const ") else "ptr"
    raise AssertionError(f"unmapped C type {t!r}")


def _zig_type(t: str) -> str:
    t = t.strip()
    table = {
        "c_int": "int", "f32": "f32", "usize": "usize", "void": "void", "*usize": "*usize", "*c_int": "*int",
        "[*c]u8": "[*c]u8", "?*const anyopaque": "cptr", "?*anyopaque": "ptr",
    }
    if t not in table:
        raise AssertionError(f"unmapped Zig type {t!r}")
    return table[t]


def c_decls():
    src = _strip_c_comments(open(HEADER).read())
    out = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(hip_\w+)\s*\(([^)]*)\)\s*;", src):
        ret, name, args = m.group(1), m.group(2), m.group(3).strip()
        ret = ret.split("\n")[-1].strip()
        types = []
        if args and args != "void":
            for a in args.split(","):
                a = " ".join(a.split())
                a = re.sub(r"\b\w+$", "", a)  # drop the parameter name
                types.append(_c_type(a))
        rt = _c_type(ret)
        out[name] = ("cptr" if rt in ("cptr", "ptr") and ret.strip().startswith("void") else rt, types)
    return out


def zig_externs(path):
    src = re.sub(r"//[^\n]*", " ", open(path).read())
    out = {}
    for m in re.finditer(r"extern\s+fn\s+(\w+)\s*\(([^)]*)\)\s*([^;{]+);", src):
        name, args, ret = m.group(1), m.group(2), m.group(3)
        types = []
        for a in args.split(","):
            a = a.strip()
            if not a:
                continue
            pname, ptype = a.split(":", 1)
            types.append(_zig_type(ptype))
        rt = _zig_type(ret)
        out[name] = ("cptr" if rt == "ptr" else rt, types)
    return out


@pytest.mark.parametrize("fname", ["attention_hip.zig", "hip_context.zig"])
def test_zig_externs_match_c_header(fname):
    c = c_decls()
    z = zig_externs(os.path.join(ZIG, fname))
    assert z, f"no externs parsed from {fname}"
    for name, (ret, args) in z.items():
        assert name in c, f"{fname}: {name} is not declared in llmgen_attn.h"
        c_ret, c_args = c[name]
        assert len(args) == len(c_args), f"{name}: {len(args)} Zig arguments, {len(c_args)} in C"
        assert args == c_args, f"{name}: argument types differ\n zig {args}\n   c {c_args}"
        # void * returns: Zig ?*anyopaque
        assert ret == c_ret or (ret == "cptr" and c_ret == "cptr"), f"{name}: return {ret} vs {c_ret}"


def test_every_c_entry_point_is_bound_in_zig():
    c = c_decls()
    bound = set()
    for f in ("attention_hip.zig", "hip_context.zig"):
        bound |= set(zig_externs(os.path.join(ZIG, f)))
    skip = {"hip_set_stream", "hip_get_stream", "hip_timer_create", "hip_timer_record", "hip_timer_elapsed_ms",
            "hip_timer_destroy"}  # host conveniences for non-Zig callers (no reference counterpart)
    missing = sorted(set(c) - bound - skip)
    assert not missing, f"declared in llmgen_attn.h but not bound in zig/: {missing}"


def test_c_parser_sees_the_reference_shaped_launchers():
    c = c_decls()
    assert c["hip_attn_decode"][1] == ["ptr", "cptr", "cptr", "cptr", "cptr", "cptr", "int", "int", "int", "int",
                                       "int", "int", "f32", "ptr", "ptr", "int", "int"]
    assert c["hip_attn_prefill_tile"] == ("int", [])
    assert c["hip_graph_end"][0] == "cptr"


def test_execute_body_issues_the_operator_calls():
    """PagedAttentionImpl.execute reads g_step / kvOf and issues store_kv + prefill (with the single-row count), or
    the fused decode."""
    src = open(os.path.join(ZIG, "attention_hip.zig")).read()
    body = src[src.index("pub const PagedAttentionImpl"):]
    assert "common.kvOf(out.layer_id)" in body and "common.g_step" in body
    for call in ("hip_store_kv(", "hip_attn_prefill_rows(", "hip_attn_decode_store_kv("):
        assert call in body, call
    assert "pub const FlashAttentionImpl = PagedAttentionImpl;" in src
    # prefill passes the step's single-row count (read from g_step when the engine records it)
    assert _call_args(body, "hip_attn_prefill_rows")[-1].strip() == "singleRowsOf(st)"
    assert '@hasField(@TypeOf(st.*), "single_rows")' in src
    # every call passes every argument the C declaration has
    for name in ("hip_attn_decode_store_kv", "hip_store_kv", "hip_attn_prefill_rows"):
        assert len(_call_args(body, name)) == len(c_decls()[name][1]), name


def _call_args(src, name):
    """Top-level arguments of the first call `name(...)` in src (commas inside nested parentheses kept)."""
    i = src.index(name + "(") + len(name) + 1
    depth, cur, args = 0, "", []
    while True:
        ch = src[i]
        i += 1
        if ch == "(":
            depth += 1
        elif ch == ")":
            if depth == 0:
                break
            depth -= 1
        if ch == "," and depth == 0:
            args.append(cur)
            cur = ""
        else:
            cur += ch
    args.append(cur)
    return [a for a in args if a.strip()]


def test_step_hints_zig_mirrors_the_cpp_fill_meta():
    """zig/step_hints.zig (what the Zig executor adds to fillMeta / bindStep) has the two functions, with the
    C++ slice's ordering key (single-row tiles first, then keys a tile needs = ctx - q_len + min(q0 + tile,
    q_len)) and a stable sort."""
    src = open(os.path.join(ZIG, "step_hints.zig")).read()
    assert "pub fn singleRows(" in src and "pub fn sortTilesLightestFirst(" in src
    assert "ctx[s] - q_len + tile_end" in src and "@min(tq0[i] + @as(i32, @intCast(pf_tile)), q_len)" in src
    assert "(multi << 32) + keys" in src  # single-row tiles first
    assert "> key" in src  # strictly greater: equal keys keep their order (stable)
