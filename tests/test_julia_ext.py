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
