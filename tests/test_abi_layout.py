"""The PJRT v0.55 structs that jaxlib and this plugin exchange, pinned byte
for byte.  jaxlib reads the PJRT_Api table and every *_Args struct by offset,
so `mccl-jax_amd/src/pjrt/api/pjrt_abi.h` (a restatement written as an
X-macro list) must have the layout of XLA's header at the commit the
reference pins (third_party/xla/pjrt/c/pjrt_c_api.h, PROVENANCE.md:6-8;
the table is pjrt_c_api.h:2125-2253).

A C probe is generated from pjrt_abi.h itself: for every struct it spells
out, sizeof and offsetof of every member (anonymous-union members included)
and the minimal struct_size (offset + size of the last member, what
PJRT_DEFINE_STRUCT_TRAITS defines); for PJRT_Api, the offset of all 100
slots; for every enum, every enumerator's value.  The probe is compiled
against pjrt_abi.h and, when /root/reference is present, against the
reference's header; both outputs must be identical.  The reference's output
is kept as a fixture (tests/golden/pjrt_abi_layout.txt) so the check also
runs where the reference is absent.  CPU only (gcc)."""

import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ABI_H = os.path.join(ROOT, "mccl-jax_amd", "src", "pjrt", "api", "pjrt_abi.h")
REF_H = "/root/reference/third_party/xla/pjrt/c/pjrt_c_api.h"
FIXTURE = os.path.join(ROOT, "tests", "golden", "pjrt_abi_layout.txt")


def _strip_comments(t):
    t = re.sub(r"/\*.*?\*/", "", t, flags=re.S)
    return re.sub(r"//[^\n]*", "", t)


def _balanced(text, start):
    """Index one past the bracket that closes the one at text[start]."""
    pairs = {"(": ")", "{": "}"}
    open_c = text[start]
    close_c = pairs[open_c]
    depth = 0
    for i in range(start, len(text)):
        if text[i] == open_c:
            depth += 1
        elif text[i] == close_c:
            depth -= 1
            if depth == 0:
                return i + 1
    raise ValueError("unbalanced")


def _fields(body):
    """Member names of a struct body, in order (anonymous unions flattened)."""
    body = body.replace("MI_ARGS_HEAD", "size_t struct_size; PJRT_Extension_Base* extension_start;")
    body = re.sub(r"union\s*\{", "", body)
    body = body.replace("}", "")
    names = []
    for decl in body.split(";"):
        decl = decl.strip()
        if not decl:
            continue
        m = re.search(r"\(\s*\*\s*(\w+)\s*\)", decl)
        if m:
            names.append(m.group(1))
            continue
        names.append(re.findall(r"\w+", decl)[-1])
    return names


def parse_abi(text):
    text = _strip_comments(text)
    slots_def = re.search(r"#define MI_PJRT_SLOTS\(F, V\)(.*?)\n\s*\n", text, flags=re.S).group(1)
    slots = re.findall(r"\b[FV]\((\w+)\)", slots_def)
    kept, in_macro = [], False
    for line in text.split("\n"):  # drop macro definitions (with their continuation lines)
        if line.lstrip().startswith("#define") or in_macro:
            in_macro = line.rstrip().endswith("\\")
            continue
        kept.append(line)
    text = "\n".join(kept)
    structs = {}
    for m in re.finditer(r"\bMI_ARGS\(", text):
        end = _balanced(text, m.end() - 1)
        inner = text[m.end():end - 1]
        name, body = inner.split(",", 1)
        structs[name.strip()] = ["struct_size", "extension_start"] + _fields(body)
    for m in re.finditer(r"typedef struct (\w+)\s*\{", text):
        end = _balanced(text, m.end() - 1)
        structs[m.group(1)] = _fields(text[m.end():end - 1])
    enums = {}
    for m in re.finditer(r"typedef enum\s*\{", text):
        end = _balanced(text, m.end() - 1)
        name = re.match(r"\s*(\w+)", text[end:]).group(1)
        enums[name] = [e.split("=")[0].strip() for e in text[m.end():end - 1].split(",") if e.strip()]
    return structs, enums, slots


def probe_source(header, structs, enums, slots):
    lines = [f'#include "{header}"', "#include <stdio.h>", "#include <stddef.h>",
             "#define SZ(s) printf(\"sizeof %s %zu\\n\", #s, sizeof(s))",
             "#define OFF(s, f) printf(\"offsetof %s.%s %zu\\n\", #s, #f, offsetof(s, f))",
             "#define MIN(s, f) printf(\"struct_size %s %zu\\n\", #s, offsetof(s, f) + sizeof(((s*)0)->f))",
             "#define EN(e) printf(\"enum %s %ld\\n\", #e, (long)(e))",
             "int main(void) {"]
    for s, fs in sorted(structs.items()):
        lines.append(f"  SZ({s});")
        for f in fs:
            lines.append(f"  OFF({s}, {f});")
        lines.append(f"  MIN({s}, {fs[-1]});")
    lines.append("  SZ(PJRT_Api);")
    for sl in slots:
        lines.append(f"  OFF(PJRT_Api, PJRT_{sl});")
    for _, es in sorted(enums.items()):
        for e in es:
            lines.append(f"  EN({e});")
    lines.append("  return 0;\n}")
    return "\n".join(lines) + "\n"


def run_probe(tmp_path, header, tag):
    structs, enums, slots = parse_abi(open(ABI_H).read())
    src = tmp_path / f"probe_{tag}.c"
    src.write_text(probe_source(header, structs, enums, slots))
    exe = tmp_path / f"probe_{tag}"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-o", str(exe), str(src)], check=True,
                   capture_output=True, text=True)
    return subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout


def test_parser_sees_every_struct_and_slot():
    structs, enums, slots = parse_abi(open(ABI_H).read())
    assert len(slots) == 100 and len(set(slots)) == 100
    assert "PJRT_LoadedExecutable_Execute_Args" in structs and "PJRT_NamedValue" in structs
    assert structs["PJRT_Client_CreateViewOfDeviceBuffer_Args"][-4:] == [
        "on_delete_callback", "on_delete_callback_arg", "stream", "buffer"]
    assert "string_value" in structs["PJRT_NamedValue"] and "tiled" in structs["PJRT_Buffer_MemoryLayout"]
    assert len(structs) >= 90 and "PJRT_Buffer_Type" in enums


def test_layout_matches_pinned_reference_header(tmp_path):
    ours = run_probe(tmp_path, ABI_H, "ours")
    if os.path.exists(REF_H):
        ref = run_probe(tmp_path, REF_H, "ref")
        if not os.path.exists(FIXTURE) or open(FIXTURE).read() != ref:
            with open(FIXTURE, "w") as f:
                f.write(ref)
    else:
        if not os.path.exists(FIXTURE):
            pytest.skip("neither the reference header nor the layout fixture is present")
        ref = open(FIXTURE).read()
    ours_l, ref_l = ours.splitlines(), ref.splitlines()
    diff = [(a, b) for a, b in zip(ours_l, ref_l) if a != b]
    assert len(ours_l) == len(ref_l) and not diff, diff[:10]
    assert "sizeof PJRT_Api 840" in ref_l
