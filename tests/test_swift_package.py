"""CPU: the SwiftPM package under animaxs_amd/swift is bound to the same C boundary the C layout
test compiles.  Its module map must name include/anima_hip.h itself (no copy that could drift),
every anima_* function and ANIMA_* constant the Swift wrappers use must be declared there, and
every C struct the wrappers build with a memberwise initialiser must list the struct's fields in
declaration order (Swift imports C structs with exactly that initialiser).  No Swift toolchain
exists in this image, so the package is checked against the header, not compiled."""

from __future__ import annotations

import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "animaxs_amd", "swift")
HEADER = os.path.join(ROOT, "include", "anima_hip.h")
SOURCES = os.path.join(PKG, "Sources", "AnimaHIP")


def _header_text() -> str:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def _swift_text() -> str:
    parts = []
    for name in sorted(os.listdir(SOURCES)):
        assert name.endswith(".swift"), name
        parts.append(re.sub(r"//[^\n]*", " ", open(os.path.join(SOURCES, name)).read()))
    return "\n".join(parts)


def _struct_fields(header: str, name: str) -> list[str]:
    m = re.search(r"typedef struct %s \{(.*?)\} %s;" % (name, name), header, flags=re.S)
    assert m, name
    fields = []
    for decl in m.group(1).split(";"):
        decl = decl.strip()
        if not decl:
            continue
        # "anima_buffer packed" / "int64_t rows" / "const int32_t* key_lengths"
        fields.append(re.findall(r"[A-Za-z_][A-Za-z_0-9]*", decl)[-1])
    return fields


def test_module_map_names_the_repository_header():
    mm_dir = os.path.join(PKG, "Sources", "CAnimaHIP")
    text = open(os.path.join(mm_dir, "module.modulemap")).read()
    headers = re.findall(r'header\s+"([^"]+)"', text)
    assert len(headers) == 1
    assert os.path.realpath(os.path.join(mm_dir, headers[0])) == os.path.realpath(HEADER)
    assert re.search(r'link\s+"anima_hip"', text)
    # the C layout test compiles that same header
    assert "anima_hip.h" in open(os.path.join(ROOT, "tests", "c", "abi_layout.c")).read()


def test_swift_wrappers_use_only_declared_symbols():
    header = _header_text()
    declared_fns = set(re.findall(r"\b(anima_[a-z0-9_]+)\s*\(", header))
    # enum constants, and integer macros (Swift imports a literal #define as a constant)
    declared_consts = set(re.findall(r"\b(ANIMA_[A-Z0-9_]+)\s*=", header))
    declared_consts |= set(re.findall(r"#define (ANIMA_[A-Z0-9_]+)\s+(?:0x[0-9A-Fa-f]+|[0-9]+)u?\s", header))
    declared_types = set(re.findall(r"typedef (?:struct|enum) (anima_[a-z0-9_]+)", header))
    swift = _swift_text()
    # calls and function references (an entry point passed as a closure) alike
    used_fns = set(re.findall(r"\b(anima_[a-z0-9_]+)\b", swift)) - declared_types
    used_consts = set(re.findall(r"\b(ANIMA_[A-Z0-9_]+)\b", swift))
    assert used_fns, "no C calls found"
    assert used_fns <= declared_fns, sorted(used_fns - declared_fns)
    assert used_consts <= declared_consts, sorted(used_consts - declared_consts)
    # the three reference surfaces and their entry points are all bound
    for fn in ("anima_attention_create", "anima_attention_encode", "anima_attention_execute",
               "anima_attention_max_score_scratch_bytes", "anima_linear_create", "anima_linear_encode",
               "anima_linear_execute", "anima_dequant_w4", "anima_dequant_w4_matrix", "anima_dequant_w8",
               "anima_dequant_w8_matrix", "anima_fp16_to_float32"):
        assert fn in used_fns, fn
    for cls in ("class AttentionExecutor", "class LinearExecutor", "enum QuantDecoders",
                "struct QuantizedLinearWeightBuffers", "enum AttentionNumerics", "enum AttentionInputLayout",
                "enum DiTAttentionBackend", "enum DiTLinearBackend", "enum DiTLinearFamily"):
        assert cls in swift, cls


def test_memberwise_initialisers_follow_the_header_field_order():
    header = _header_text()
    swift = _swift_text()
    checked = 0
    for m in re.finditer(r"\b(anima_[a-z0-9_]+)\(([^()]*(?:\([^()]*\)[^()]*)*)\)", swift):
        name, body = m.group(1), m.group(2)
        if not re.search(r"typedef struct %s \{" % name, header):
            continue
        labels = re.findall(r"(?:^|,)\s*([a-z_][a-z0-9_]*)\s*:", body)
        if not labels:
            continue                      # the zero initialiser anima_x()
        assert labels == _struct_fields(header, name), (name, labels)
        checked += 1
    assert checked >= 3, checked
