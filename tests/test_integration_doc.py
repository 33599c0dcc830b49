"""The Swift binding in the integration guide (the ```swift blocks of the
Markdown file at DOC) against the C headers and the reference's public Swift
surface (CPU only; nothing is compiled or launched).

The binding is documentation a maintainer pastes into the reference package,
so nothing else checks it: these tests fail when it calls a `gd_*` function
the headers do not declare or with the wrong number of arguments, names a
`GD_*` constant that does not exist, leaves out a constructor flag the header
defines, or drifts from the reference signatures it must keep
(DeBERTa.swift:7-58, 188-272; FusedKernels.swift:157-286).
"""

import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
DOC = ROOT / "INTEGRATION.md"
HEADERS = [ROOT / "include" / h for h in ("gliner_decide.h", "gliner_decide_frontend.h", "gliner_decide_diag.h")]


def swift_blocks():
    return re.findall(r"```swift\n(.*?)```", DOC.read_text(), flags=re.S)


def swift_code():
    return "\n".join(swift_blocks())


def _strip_c_comments(text):
    return re.sub(r"/\*.*?\*/", " ", text, flags=re.S)


def _top_level_split(args):
    """Splits an argument list at commas outside brackets and string literals."""
    parts, depth, cur, in_str = [], 0, [], False
    for i, ch in enumerate(args):
        if in_str:
            cur.append(ch)
            if ch == '"' and args[i - 1] != "\\":
                in_str = False
            continue
        if ch == '"':
            in_str = True
        elif ch in "([{":
            depth += 1
        elif ch in ")]}":
            depth -= 1
        elif ch == "," and depth == 0:
            parts.append("".join(cur).strip())
            cur = []
            continue
        cur.append(ch)
    tail = "".join(cur).strip()
    if tail:
        parts.append(tail)
    return parts


def _call_args(text, start):
    """Argument list of the call whose '(' is at text[start]."""
    depth = 0
    for j in range(start, len(text)):
        if text[j] == "(":
            depth += 1
        elif text[j] == ")":
            depth -= 1
            if depth == 0:
                return text[start + 1:j]
    raise AssertionError("unbalanced call at %r" % text[start:start + 60])


def header_prototypes():
    """{function name: parameter count} of every gd_* prototype in the headers."""
    protos = {}
    for h in HEADERS:
        text = _strip_c_comments(h.read_text())
        for m in re.finditer(r"\b(gd_\w+)\s*\(", text):
            # a declaration: preceded by a return type on the same statement
            line_start = text.rfind("\n", 0, m.start()) + 1
            prefix = text[line_start:m.start()]
            if not re.search(r"\b(int|void|char|int64_t|const)\b[\s*]*$", prefix):
                continue
            params = _call_args(text, m.end() - 1).strip()
            protos[m.group(1)] = 0 if params in ("", "void") else len(_top_level_split(params))
    return protos


def header_constants():
    names = set()
    for h in HEADERS:
        text = _strip_c_comments(h.read_text())
        names |= set(re.findall(r"#define\s+(GD_\w+)", text))
        for body in re.findall(r"enum\s+\w*\s*\{(.*?)\}", text, flags=re.S):
            names |= set(re.findall(r"\b(GD_\w+)\s*(?:=|,|$)", body))
    return names


def header_types():
    names = set()
    for h in HEADERS:
        text = _strip_c_comments(h.read_text())
        names |= set(re.findall(r"typedef\s+(?:struct|enum)\s+\w*\s*(?:\{.*?\})?\s*(gd_\w+)\s*;", text, flags=re.S))
    return names


def test_doc_has_the_bindings():
    code = swift_code()
    assert "public final class GLiNERDecideClassifier" in code
    assert "public final class FusedKernels" in code
    assert "public struct DecisionInput" in code


def test_every_gd_call_is_declared_with_its_arity():
    protos = header_prototypes()
    assert "gd_classifier_create" in protos and protos["gd_classifier_create"] == 5
    code = swift_code()
    calls = list(re.finditer(r"\b(gd_\w+)\s*\(", code))
    assert len(calls) >= 15
    types = header_types()
    for m in calls:
        name = m.group(1)
        if name in types:  # a C struct's zero initialiser, e.g. gd_config()
            assert _call_args(code, m.end() - 1).strip() == "", name
            continue
        assert name in protos, f"{name} is called by the Swift binding but declared in no header"
        n = len(_top_level_split(_call_args(code, m.end() - 1)))
        assert n == protos[name], f"{name}: the binding passes {n} arguments, the header declares {protos[name]}"


def test_every_gd_constant_and_type_exists():
    code = swift_code()
    consts = header_constants()
    for name in set(re.findall(r"\b(GD_[A-Z0-9_]+)\b", code)):
        assert name in consts, f"{name} is used by the Swift binding but defined in no header"
    types = header_types()
    for name in set(re.findall(r"\b(gd_[a-z0-9_]+)\b", code)) - set(header_prototypes()):
        assert name in types, f"{name} is neither a declared function nor a declared type"


def test_every_constructor_flag_is_bound():
    text = _strip_c_comments((ROOT / "include" / "gliner_decide.h").read_text())
    flags = set(re.findall(r"#define\s+(GD_USE_\w+)", text))
    assert flags == {"GD_USE_FUSED_KERNELS", "GD_USE_COMPILED_GRAPH", "GD_USE_GENERIC_ATTENTION",
                     "GD_USE_CUSTOM_RELATIVE_KERNEL", "GD_USE_FUSED_ATTENTION_KERNEL"}
    code = swift_code()
    for f in flags:
        assert f in code, f"header flag {f} is missing from the Swift binding"


def _init_params(code, owner):
    """(label, type, default) of `owner`'s public init taking weightsURL."""
    m = re.search(r"public init\(\s*weightsURL:", code)
    assert m, "no init(weightsURL:...) in the binding"
    params = _top_level_split(_call_args(code, m.start() + len("public init")))
    out = []
    for p in params:
        pm = re.fullmatch(r"(\w+)\s*:\s*([\w.]+)\s*(?:=\s*([\w.]+))?", p.strip())
        assert pm, p
        out.append(pm.groups())
    return out


def test_classifier_init_keeps_the_reference_signature():
    # DeBERTa.swift:188-196
    expected = [("weightsURL", "URL", None), ("configuration", "DeBERTaV2Configuration", ".default"),
                ("useFusedKernels", "Bool", "false"), ("useCompiledGraph", "Bool", "false"),
                ("useFastAttention", "Bool", "true"), ("useCustomRelativeKernel", "Bool", "false"),
                ("useFusedAttentionKernel", "Bool", "false")]
    assert _init_params(swift_code(), "GLiNERDecideClassifier") == expected


def test_flags_map_to_their_parameters():
    code = swift_code()
    for cond, flag in [("useFusedKernels", "GD_USE_FUSED_KERNELS"), ("useCompiledGraph", "GD_USE_COMPILED_GRAPH"),
                       ("!useFastAttention", "GD_USE_GENERIC_ATTENTION"),
                       ("useCustomRelativeKernel", "GD_USE_CUSTOM_RELATIVE_KERNEL"),
                       ("useFusedAttentionKernel", "GD_USE_FUSED_ATTENTION_KERNEL")]:
        assert re.search(r"if\s+" + re.escape(cond) + r"\s*\{\s*flags\s*\|=\s*" + flag + r"\s*\}", code), flag


def test_classify_and_result_types_keep_the_reference_surface():
    code = swift_code()
    # DeBERTa.swift:244-247
    assert re.search(r"public func classify\(_ input: DecisionInput, collectProfile: Bool = false\) -> InferenceResult",
                     code)
    # DeBERTa.swift:14-20
    body = re.search(r"public struct InferenceResult \{(.*?)\n\}", code, flags=re.S).group(1)
    for field in ("public let logits:", "public let wallNanoseconds: UInt64", "public let events: [ProfileEvent]",
                  "public var wallMilliseconds: Double"):
        assert field in body, field
    # DeBERTa.swift:7-12
    body = re.search(r"public struct ProfileEvent[^{]*\{(.*?)\n\}", code, flags=re.S).group(1)
    for field in ("public let name: String", "public let nanoseconds: UInt64", "public var milliseconds: Double"):
        assert field in body, field
    # DeBERTa.swift:22-58
    body = re.search(r"public struct DecisionInput \{(.*?)\n\}\n", code, flags=re.S).group(1)
    for field in ("inputIDs", "attentionMask", "markerIndices", "markerMask"):
        assert re.search(r"public let " + field + r":", body), field
    assert re.search(r"public init\(inputIDs: [^,]+, attentionMask: [^,]+,\s*markerIndices: [^,]+, markerMask: [^)]+\)",
                     body)
    assert "public init(url: URL) throws" in body
    assert "Input safetensors must contain input_ids, attention_mask, marker_indices, and marker_mask" in body


def test_classify_runs_profiled_and_packed_entry_points():
    code = swift_code()
    run = re.search(r"private func run\(.*?\n    \}\n", code, flags=re.S).group(0)
    assert "gd_classifier_classify_profiled" in run and "gd_classifier_classify_packed" in run
    assert "hipMemcpyDeviceToHost" in run


def test_fused_kernels_shim_keeps_method_names():
    code = swift_code()
    # FusedKernels.swift:157-286
    for name in ("fusedAttention", "relativeBias", "residualLayerNorm"):
        assert re.search(r"public func " + name + r"\(", code), name


def test_no_stale_unsupported_text():
    text = DOC.read_text()
    assert "exits with `GD_ERR_UNSUPPORTED`" not in text
    assert "need no flag" not in text
    assert "is the only\n  attention path" not in text and "only attention path" not in text


def test_total_tokens_rule_matches_row_extents():
    """The Swift totalTokens loop restates decode.row_extents; run the same
    rule in Python over a case with masked, out-of-range and late markers."""
    import numpy as np
    from gliner_decide.decode import row_extents
    mask = np.array([[1, 1, 0, 0, 0, 0], [0, 0, 0, 0, 0, 0], [1, 1, 1, 1, 1, 1], [1, 0, 0, 0, 0, 0]], np.float16)
    markers = np.array([[[1, 4]], [[9, 0]], [[2, 3]], [[-1, 2]]], np.int32)
    mmask = np.array([[[1, 1]], [[1, 0]], [[1, 1]], [[1, 0]]], np.float32)

    def swift_rule():  # line for line the loop in DecisionInput.totalTokens
        b, l = mask.shape
        slots = markers.size // b
        total = 0
        for r in range(b):
            extent = 0
            for p in range(l):
                if mask.reshape(-1)[r * l + p] > 0:
                    extent = p + 1
            for s in range(slots):
                if mmask.reshape(-1)[r * slots + s] > 0:
                    m = int(markers.reshape(-1)[r * slots + s])
                    extent = max(extent, m + 1 if 0 <= m < l else 1)
            total += extent
        return total

    ext = row_extents(mask, markers, mmask)
    assert list(ext) == [5, 1, 6, 1]
    assert swift_rule() == int(ext.sum()) == 13
    code = swift_code()
    assert "extent = max(extent, (m >= 0 && m < l) ? m + 1 : 1)" in code
