"""CPU checks of the Julia extension (julia/ext/FlashMaxSimHIPExt.jl) against the C
header, without Julia: every ``ccall`` names a declared symbol and passes the
declared number of arguments, in the declared order and of compatible types;
the buffer-taking boundary methods only accept the Float32 buffers the library
writes; the package fragment wires the extension as a weak dependency; and the
at-rest Int8Index reader's header patterns find the fields of a file written by
the Python host."""
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "flashmaxsim_hip.h")
JL_DIR = os.path.join(ROOT, "flashmaxsim.jl_amd", "julia")
EXT = os.path.join(JL_DIR, "ext", "FlashMaxSimHIPExt.jl")
PROJECT = os.path.join(JL_DIR, "Project.toml")


# ---- C header ---------------------------------------------------------------------

def header_decls():
    """name -> (return type, [(param type, param name)])."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = re.sub(r"//[^\n]*", " ", text)
    text = re.sub(r"(?m)^\s*#.*$", " ", text)        # preprocessor lines
    text = re.sub(r"\btypedef\b[^;]*;", " ", text)
    decls = {}
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(fms_\w+)\s*\(([^;{]*?)\)\s*;", text):
        ret, name, params = " ".join(m.group(1).split()), m.group(2), m.group(3).strip()
        plist = []
        if params and params != "void":
            for p in params.split(","):
                p = " ".join(p.split())
                pm = re.match(r"(.*?)([A-Za-z_]\w*)$", p)
                plist.append((pm.group(1).replace(" *", "*").strip(), pm.group(2)))
        decls[name] = (ret, plist)
    return decls


# ---- Julia ccall parser --------------------------------------------------------------

def split_top(s):
    """Split s on commas at nesting depth 0 of (), [], {}."""
    out, depth, cur = [], 0, []
    for ch in s:
        if ch in "([{":
            depth += 1
        elif ch in ")]}":
            depth -= 1
        if ch == "," and depth == 0:
            out.append("".join(cur).strip())
            cur = []
        else:
            cur.append(ch)
    if "".join(cur).strip():
        out.append("".join(cur).strip())
    return out


def ccalls(text):
    """[(symbol, return type, [arg types], [arg expressions], line)] for every ccall."""
    text_nc = re.sub(r"#[^\n]*", "", text)
    found = []
    for m in re.finditer(r"ccall\(", text_nc):
        i, depth = m.end(), 1
        while depth:
            depth += {"(": 1, ")": -1}.get(text_nc[i], 0)
            i += 1
        parts = split_top(text_nc[m.end():i - 1])
        sym = re.match(r"\(\s*:(\w+)\s*,\s*libfms\s*\)", parts[0])
        assert sym, parts[0]
        types = parts[2].strip()
        assert types.startswith("(") and types.endswith(")"), types
        tlist = split_top(types[1:-1])
        line = text_nc[:m.start()].count("\n") + 1
        found.append((sym.group(1), parts[1].strip(), tlist, parts[3:], line))
    return found


def c_ptr(ctype):
    return ctype.endswith("*")


TYPE_OK = {
    "Int32": lambda c: c in ("int32_t", "fms_status"),
    "Int64": lambda c: c == "int64_t",
    "Float32": lambda c: c == "float",
    "Cint": lambda c: c == "int",
    "Cstring": lambda c: c == "const char*",
    "Ptr{Cvoid}": c_ptr,
}


def test_every_ccall_matches_the_header():
    decls = header_decls()
    calls = ccalls(open(EXT).read())
    assert len(calls) >= 20
    seen = set()
    for sym, ret, tlist, args, line in calls:
        where = f"{os.path.basename(EXT)}:{line} {sym}"
        assert sym in decls, f"{where}: not declared in the header"
        cret, params = decls[sym]
        seen.add(sym)
        assert TYPE_OK[ret](cret), f"{where}: return {ret} vs {cret}"
        assert len(tlist) == len(params), f"{where}: {len(tlist)} argument types, header has {len(params)}"
        assert len(args) == len(params), f"{where}: {len(args)} arguments, header has {len(params)}"
        names = {n for _, n in params}
        for k, ((ctype, cname), jtype, expr) in enumerate(zip(params, tlist, args)):
            at = f"{where} argument {k + 1} ({cname})"
            assert jtype in TYPE_OK, f"{at}: unexpected Julia type {jtype}"
            assert TYPE_OK[jtype](ctype), f"{at}: {jtype} vs {ctype}"
            if c_ptr(ctype) and cname != "stream":
                pm = re.fullmatch(r"dptr\((\w+)\)", expr)
                assert expr == "C_NULL" or pm, f"{at}: pointer argument {expr!r}"
                if pm:
                    assert pm.group(1) == cname, f"{at}: passes {pm.group(1)}"
            elif cname == "stream":
                assert expr == "stream_ptr()", f"{at}: {expr!r}"
            elif re.fullmatch(r"[A-Za-z_]\w*", expr):
                # a bare variable in a size slot must not be another parameter's name
                assert expr == cname or expr not in names, f"{at}: passes {expr}"
            if cname == "idx_bytes":
                assert "sizeof(eltype(idx" in expr, f"{at}: {expr!r}"
            if cname in ("qs_dtype", "ds_dtype", "dtype"):
                assert expr == cname or re.fullmatch(r"(dtype_code|scale_code)\(.+\)", expr), \
                    f"{at}: {expr!r}"
    boundary = {"fms_launch_pair_scan", "fms_launch_paired_scan", "fms_launch_candidates_scan",
                "fms_inbatch_device_scan", "fms_launch_packed_scan", "fms_launch_varlen_scan",
                "fms_launch_int8_pair_scan", "fms_launch_int8_paired_scan",
                "fms_launch_int8_candidates_scan", "fms_int8_quantize", "fms_arch_supported",
                "fms_pair_pullback", "fms_paired_pullback", "fms_inbatch_pullback",
                "fms_candidates_pullback", "fms_packed_pullback", "fms_varlen_pullback",
                "fms_launch_packed_multi_scan", "fms_topk", "fms_status_string"}
    assert boundary <= seen, sorted(boundary - seen)


def method_signatures(text, pattern):
    """(name, signature text) of every `function FlashMaxSim.<name>(...) where ...`."""
    out = []
    for m in re.finditer(r"function FlashMaxSim\.(" + pattern + r")\(", text):
        i, depth = m.end(), 1
        while depth:
            depth += {"(": 1, ")": -1}.get(text[i], 0)
            i += 1
        tail = text[i:i + 200].split("\n")[0]
        out.append((m.group(1), text[m.end():i - 1], tail))
    return out


def test_buffer_taking_methods_require_float32_buffers():
    """The reference allocates partial / S as dot_accum(T) (kernels_forward.jl:16-21):
    BFloat16 for BFloat16 features.  The library writes Float32, so a boundary method
    that receives the reference's buffers must only match Float32 ones."""
    text = open(EXT).read()
    sigs = method_signatures(text, r"launch_\w+_scan!|inbatch_device_scan!")
    assert {s[0] for s in sigs} == {
        "launch_pair_scan!", "launch_paired_scan!", "launch_candidates_scan!",
        "inbatch_device_scan!", "launch_packed_scan!", "launch_varlen_scan!",
        "launch_int8_pair_scan!", "launch_int8_paired_scan!"}
    for name, sig, tail in sigs:
        buf = "S" if name == "inbatch_device_scan!" else "partial"
        m = re.search(r"\b" + buf + r"::ROC(?:Vector|Matrix|Array)\{Float32", sig)
        assert m, f"{name}: {buf} is not required to be a Float32 device array"
        assert "AnyFeature" not in tail and "BFloat16" not in sig, name
        if "int8" not in name:
            assert "T<:ScanFeature" in tail, f"{name}: feature type not limited to Float16/Float32"


def test_bfloat16_reaches_the_library_only_through_drivers():
    text = open(EXT).read()
    assert re.search(r"const ScanFeature = Union\{Float16, Float32\}", text)
    sigs = method_signatures(text, r"\w+_forward_ka")
    assert {s[0] for s in sigs} == {"pair_forward_ka", "paired_forward_ka", "inbatch_forward_ka",
                                    "candidates_forward_ka", "packed_forward_ka",
                                    "varlen_forward_ka"}
    for name, sig, tail in sigs:
        assert "T<:AnyFeature" in tail, name
    # every driver allocates its own Float32 outputs and passes no partial buffer
    for m in re.finditer(r"function FlashMaxSim\.(\w+_forward_ka)\(.*?\nend\n", text, flags=re.S):
        body = m.group(0)
        assert "AMDGPU.zeros(Float32" in body, m.group(1)
        assert not re.search(r"similar\([^)]*score_eltype", body), m.group(1)
        assert re.search(r"c_\w+_scan\(dtype_code\(T\), \w+, nothing", body) or \
            "c_inbatch_scan" in body, m.group(1)


# The backend type each overridden reference method is declared on, so that
# `@invoke` with that annotation selects the reference method and never the
# extension's ROCBackend one.
REFERENCE_BACKEND = {
    # src/forward_pair.jl:130, src/forward_layouts.jl:139,306, src/packed.jl,
    # src/quant.jl: launch_*_scan!(backend::GPU, ...) run the KA tile kernels
    "launch_pair_scan!": "KAGPU", "launch_paired_scan!": "KAGPU",
    "launch_candidates_scan!": "KAGPU", "launch_packed_scan!": "KAGPU",
    "launch_varlen_scan!": "KAGPU", "launch_int8_pair_scan!": "KAGPU",
    "launch_int8_paired_scan!": "KAGPU",
    # src/forward_layouts.jl:201: inbatch_device_scan!(backend, ...) untyped
    "inbatch_device_scan!": "Any",
    # src/forward_pair.jl:104, src/packed.jl:178,262: (backend::Backend, ...)
    "pair_forward_ka": "KABackend", "packed_forward_ka": "KABackend",
    "varlen_forward_ka": "KABackend",
    # src/forward_layouts.jl:112,188,272: untyped backend
    "paired_forward_ka": "Any", "inbatch_forward_ka": "Any", "candidates_forward_ka": "Any",
    # src/backward_*.jl, src/packed.jl: (::Strategy, backend, ...) untyped backend
    "pair_apply_pullback!": "Any", "paired_apply_pullback!": "Any",
    "inbatch_apply_pullback!": "Any", "candidates_apply_pullback!": "Any",
    "packed_apply_pullback!": "Any", "varlen_apply_pullback!": "Any",
}


def arg_list(sig):
    """[(name, type or None)] of a Julia signature's positional arguments."""
    out = []
    for a in split_top(sig.split(";")[0]):
        a = " ".join(a.split())
        m = re.fullmatch(r"(\w*)\s*(?:::\s*(.+))?", a)
        assert m, a
        out.append((m.group(1), m.group(2)))
    return out


def override_bodies(text, prefix=r"FlashMaxSim\."):
    """(name, signature, first body statement) of every `function FlashMaxSim.<name>(`
    (or of the plain functions `function <name>(` with prefix "")."""
    out = []
    for m in re.finditer(r"function " + prefix + r"(\w+!?)\(", text):
        i, depth = m.end(), 1
        while depth:
            depth += {"(": 1, ")": -1}.get(text[i], 0)
            i += 1
        rest = text[i:].split("\n", 1)[1]
        first = next(line.strip() for line in rest.split("\n") if line.strip())
        out.append((m.group(1), text[m.end():i - 1], first))
    return out


MAXSIM_REFERENCE_TYPES = {
    "cfg": None, "layout": None, "Q": "AbstractArray{T,3}", "D": "AbstractArray{T,3}",
    "gallery": "AbstractArray{T,3}", "idxs": "AbstractMatrix{<:Integer}",
    "qmask": "AbstractMatrix{Bool}", "dmask": "AbstractMatrix{Bool}"}


def test_every_override_falls_back_to_the_reference_off_gfx950():
    """On an AMD GPU that is not gfx950 every override keeps the reference's own
    method, as the CUDA extension does when its tensor cores are off
    (ext/FlashMaxSimCUDAExt.jl:60-66): its first statement is
    `gfx950() || return @invoke FlashMaxSim.<same method>(<same arguments>)` with the
    backend annotated as the reference method declares it."""
    text = open(EXT).read()
    bodies = override_bodies(text)
    names = {b[0] for b in bodies}
    assert set(REFERENCE_BACKEND) | {"quantize_int8_symmetric", "maxsim"} == names, names
    for name, sig, first in bodies:
        m = re.fullmatch(r"gfx950\(\) \|\| return @invoke FlashMaxSim\.(\w+!?)\((.*)\)", first)
        assert m, f"{name}: first statement {first!r}"
        assert m.group(1) == name, f"{name}: invokes {m.group(1)}"
        declared = [n for n, _ in arg_list(sig)]
        invoked = arg_list(m.group(2))
        assert [n for n, _ in invoked] == declared, f"{name}: {invoked} vs {declared}"
        if name == "quantize_int8_symmetric":
            assert invoked == [("X", "AbstractArray{T}")], invoked
            continue
        if name == "maxsim":
            # src/dispatch.jl:80-85, 121-125, 160-167: the arrays as the reference
            # declares them, the config and layout marker as they are
            assert invoked == [(n, MAXSIM_REFERENCE_TYPES[n]) for n in declared], invoked
            continue
        bi = declared.index("backend")
        assert arg_list(sig)[bi][1] == "ROCBackend", name
        assert invoked[bi][1] == REFERENCE_BACKEND[name], f"{name}: backend::{invoked[bi][1]}"
        # only the backend (and nothing else) is widened
        assert all(t is None for k, (_, t) in enumerate(invoked) if k != bi), name
    # the extension-only entry points have no reference method: they refuse clearly
    plain = {n: f for n, _, f in override_bodies(text, prefix="")}
    for fn in ("packed_multi_scan", "topk", "int8_candidates_scan"):
        assert plain[fn].startswith("require_gfx950("), f"{fn}: {plain[fn]!r}"


# Arguments whose device pointer the library reads, and the dense types they must
# carry so that a wrapped array never reaches a raw-pointer ccall.
POINTER_ARG_TYPES = {
    "qmask": r"(DenseMask|MaybeMask)\{[123]\}",
    "dmask": r"(DenseMask|MaybeMask)\{[123]\}",
    "idx": r"DenseIndex", "idxs": r"DenseIndex",
    "inv_n": r"Union\{ROCVector\{T\}, Nothing\}",
    "P": r"DensePacked\{T\}", "Q": r"ROCArray\{T,3\}|DensePacked\{T\}",
    "D": r"ROCArray\{T,3\}|DensePacked\{T\}|Int8Index",
}
SCALAR_ARGS = {"dim", "Tq", "Td", "B", "Bq", "Bd", "C", "N", "neg", "normalize"}


def test_pointer_arguments_are_dense_device_arrays():
    """Masks, indices, inverse counts and PackedSeq storage are typed as dense
    ROCArrays in every override: a PermutedDimsArray or strided view mask
    (accepted by the reference, src/colocation.jl:18-24) then matches no
    extension method and keeps the reference path instead of reaching `dptr`."""
    text = open(EXT).read()
    assert re.search(r"^const DenseMask\{N\} = ROCArray\{Bool,N\}$", text, re.M)
    assert re.search(r"^const MaybeMask\{N\} = Union\{ROCArray\{Bool,N\}, Nothing\}$", text, re.M)
    assert re.search(r"^const DenseIndex = ROCMatrix\{<:IndexEltype\}$", text, re.M)
    assert re.search(r"^const DensePacked\{T\} = PackedSeq\{<:ROCMatrix\{T\}, <:ROCVector\{Int32\}\}$",
                     text, re.M)
    # dptr exists only for dense device arrays and nothing
    assert set(re.findall(r"^dptr\((.*?)\) =", text, re.M)) == {"x::ROCArray", "::Nothing"}
    sigs = [(n, s) for n, s, _ in override_bodies(text)]
    plain = {n: s for n, s, _ in override_bodies(text, prefix="")}
    for fn in ("int8_candidates_scan", "packed_multi_scan", "topk"):
        sigs.append((fn, plain[fn]))
    for name, sig in sigs:
        args = arg_list(sig)
        kw = sig.split(";")[1] if ";" in sig else ""
        for a in split_top(kw):
            mk = re.fullmatch(r"(\w+)\s*::\s*(.+?)\s*=.*", " ".join(a.split()))
            if mk:
                args.append((mk.group(1), mk.group(2)))
        for arg, typ in args:
            if arg in ("backend", "mode", "cfg", "layout") or arg in SCALAR_ARGS or name == "topk":
                continue
            assert typ is not None, f"{name}: argument {arg} is untyped"
            if arg in POINTER_ARG_TYPES:
                assert re.fullmatch(POINTER_ARG_TYPES[arg], typ), f"{name}: {arg}::{typ}"
            else:
                assert re.match(r"ROC(Array|Vector|Matrix)\{|Int8Index$", typ), f"{name}: {arg}::{typ}"


def test_inbatch_verb_makes_no_tape():
    """maxsim(cfg, Q, D, qmask, dmask, InBatch()) drops the tape in the reference
    (src/dispatch.jl:121-125): the override passes no args buffer (the scores-only
    kernel) and the config's normalize flag, and returns S alone."""
    text = open(EXT).read()
    m = re.search(r"function FlashMaxSim\.maxsim\((.*?)\nend\n", text, flags=re.S)
    assert m, "no maxsim override"
    body = m.group(1)
    assert "layout::FlashMaxSim.InBatch" in body and "cfg::FlashMaxSim.MaxSim{T}" in body
    assert re.search(r"c_inbatch_scan\(dtype_code\(T\), S, nothing, Q, D, qmask, dmask, dim, Tq, "
                     r"Bq, Td, Bd;\s*normalize = cfg\.normalize\)", body), body
    assert "AMDGPU.zeros(Float32, Bd, Bq)" in body and body.rstrip().endswith("S")
    assert "args" not in body


def test_paired_and_candidate_verbs_make_no_tape():
    """maxsim's paired and candidate methods (src/dispatch.jl:80-85, 160-167) drop the
    tape in the reference: the overrides pass no tape or partial buffer and the
    config's normalize flag, and return the Float32 scores alone."""
    text = open(EXT).read()
    bodies = re.findall(r"function FlashMaxSim\.maxsim\((.*?)\nend\n", text, flags=re.S)
    assert len(bodies) == 3
    paired = [b for b in bodies if "c_paired_scan" in b]
    cand = [b for b in bodies if "c_candidates_scan" in b]
    assert len(paired) == 1 and len(cand) == 1
    assert re.search(r"c_paired_scan\(dtype_code\(T\), nothing, nothing, Q, D, qmask, dmask, dim, "
                     r"Tq, Td, B, scores;\s*normalize = cfg\.normalize\)", paired[0])
    assert re.search(r"c_candidates_scan\(dtype_code\(T\), nothing, nothing, Q, gallery, idx, "
                     r"qmask, dmask,\s*dim, Tq, B, Td, N, C, scores, cfg\.neg; "
                     r"normalize = cfg\.normalize\)", cand[0])
    assert "idxs::DenseIndex" in cand[0]
    for b in paired + cand:
        assert "AMDGPU.zeros(Float32" in b and b.rstrip().endswith("scores")
        assert "args" not in b


def test_project_fragment_wires_the_extension():
    toml = open(PROJECT).read()
    weak = re.search(r"\[weakdeps\]\s*\n(.*?)(\n\[|\Z)", toml, flags=re.S)
    ext = re.search(r"\[extensions\]\s*\n(.*?)(\n\[|\Z)", toml, flags=re.S)
    assert weak and re.search(r'^AMDGPU = "21141c5a-9bdb-4563-92ae-f87d6854732e"', weak.group(1), re.M)
    assert ext and re.search(r'^FlashMaxSimHIPExt = "AMDGPU"', ext.group(1), re.M)
    # Julia finds a package extension at ext/<name>.jl
    assert os.path.exists(os.path.join(JL_DIR, "ext", "FlashMaxSimHIPExt.jl"))
    assert re.search(r"^module FlashMaxSimHIPExt$", open(EXT).read(), re.M)


# ---- the at-rest Int8Index reader ------------------------------------------------------

def julia_regex(name):
    """The pattern of `const <name> = r"..."` in the extension, as a Python regex."""
    m = re.search(r'^const ' + name + r' = r"((?:[^"\\]|\\.)*)"$', open(EXT).read(), re.M)
    assert m, name
    return re.compile(m.group(1).replace('\\"', '"'))


@pytest.mark.parametrize("scale_dtype", ["float32", "float16"])
def test_int8_index_file_reads_with_the_julia_patterns(tmp_path, scale_dtype):
    """Restates load_int8_index's parse on a file from save_int8_index: the header
    patterns find both tensors, the shapes reverse to Julia's (dim, Td, N) / (Td, N),
    and the bytes at data_offsets are the column-major arrays."""
    import torch
    from flashmaxsim import quant

    rng = np.random.default_rng(7)
    N, Td, dim = 3, 5, 8
    codes = torch.from_numpy(rng.integers(-127, 128, size=(N, Td, dim), dtype=np.int8))
    scales = torch.from_numpy(rng.random((N, Td), dtype=np.float32)).to(getattr(torch, scale_dtype))
    path = str(tmp_path / "idx.safetensors")
    quant.save_int8_index(quant.Int8Index(codes, scales), path)

    raw = open(path, "rb").read()
    n = int.from_bytes(raw[:8], "little")
    header = raw[8:8 + n].decode()
    assert julia_regex("ST_FORMAT").search(header)
    types = {"I8": np.int8, "F32": np.float32, "F16": np.float16}
    got = {}
    for which in ("CODES", "SCALES"):
        body = julia_regex("ST_ENTRY_" + which).search(header).group(1)
        dt = types[julia_regex("ST_DTYPE").search(body).group(1)]
        shape = [int(s) for s in julia_regex("ST_SHAPE").search(body).group(1).split(",") if s.strip()]
        b, e = (int(v) for v in julia_regex("ST_OFFSETS").search(body).groups())
        jl_dims = tuple(reversed(shape))
        assert e - b == int(np.prod(jl_dims)) * np.dtype(dt).itemsize
        # read! fills a column-major array of the reversed shape
        got[which] = np.frombuffer(raw[8 + n + b:8 + n + e], dtype=dt).reshape(jl_dims, order="F")
    # Julia codes[k, u, j] == torch codes[j, u, k]; scales[u, j] == torch scales[j, u]
    assert np.array_equal(got["CODES"], codes.numpy().transpose(2, 1, 0))
    assert np.array_equal(got["SCALES"], scales.numpy().T)
