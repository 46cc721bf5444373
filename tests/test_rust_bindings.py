"""The Rust crates under bindings/rust (cargo is absent here, so they are checked as text): the
`extern "C"` block of npa-hip-sys declares every function of include/npa_abi.h with the same
parameter count and return kind, every #[repr(C)] struct has the header's fields in the header's
order, and every named constant has the header's value. The safe crate npa-hip wraps each operator
of the reference's kernel crate (crates/burn_automata_kernels/src/lib.rs:40-66) in a method that
calls the matching sys function with as many arguments as that function takes."""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "npa_abi.h")
SYS = os.path.join(ROOT, "bindings", "rust", "npa-hip-sys", "src", "lib.rs")
SAFE = os.path.join(ROOT, "bindings", "rust", "npa-hip", "src", "lib.rs")


def _strip_c(text):
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    text = re.sub(r"//[^\n]*", " ", text)
    return re.sub(r"^\s*#.*$", " ", text, flags=re.M)


def _split_params(params):
    params = params.strip()
    if params in ("", "void"):
        return []
    return [p.strip() for p in params.split(",")]


def header_functions():
    text = _strip_c(open(HEADER).read())
    out = {}
    for ret, name, params in re.findall(r"([A-Za-z_][\w\s\*]*?)\b(npa_\w+)\s*\(([^;{}]*?)\)\s*;", text):
        out[name] = (" ".join(ret.split()), len(_split_params(params)))
    return out


def rust_functions():
    text = open(SYS).read()
    block = text[text.index('extern "C" {'):]
    out = {}
    for name, params, ret in re.findall(r"pub fn (npa_\w+)\s*\(([^)]*)\)\s*(->\s*[^;]+)?;", block):
        out[name] = (ret.replace("->", "").strip(), len(_split_params(params)))
    return out


def header_structs():
    text = _strip_c(open(HEADER).read())
    out = {}
    for body, name in re.findall(r"typedef struct \w+\s*\{([^}]*)\}\s*(\w+)\s*;", text):
        fields = []
        for decl in body.split(";"):
            decl = decl.strip()
            if not decl:
                continue
            # "float fx, fy" declares two fields; the type is the first declarator's prefix
            first, *rest = decl.split(",")
            fields.append(re.match(r".*?\b(\w+)\s*(\[[^\]]*\])?$", first.strip(), re.S).group(1))
            fields.extend(re.match(r"\**\s*(\w+)", r.strip()).group(1) for r in rest)
        out[name] = fields
    return out


def rust_structs():
    text = open(SYS).read()
    out = {}
    for name, body in re.findall(r"pub struct (\w+)\s*\{([^}]*)\}", text):
        out[name] = re.findall(r"pub (\w+):", body)
    return out


def header_constants():
    text = _strip_c(open(HEADER).read())
    out = dict(re.findall(r"\b(NPA_[A-Z0-9_]+)\s*=\s*(\d+)", text))
    raw = open(HEADER).read()
    for name, a, shift in re.findall(r"#define (NPA_[A-Z0-9_]+)\s+\(?(\d+)u?\s*(?:<<\s*(\d+))?", raw):
        out[name] = str(int(a) << int(shift or 0))
    return {k: int(v) for k, v in out.items()}


def rust_constants():
    out = {}
    for name, expr in re.findall(r"pub const (NPA_\w+):\s*\w+\s*=\s*([^;]+);", open(SYS).read()):
        m = re.fullmatch(r"(\d+)\s*<<\s*(\d+)", expr.strip())
        out[name] = int(m.group(1)) << int(m.group(2)) if m else int(expr)
    return out


def test_every_header_function_is_declared():
    h, r = header_functions(), rust_functions()
    assert len(h) >= 40
    assert sorted(h) == sorted(r), (set(h) ^ set(r))
    for name, (ret, count) in h.items():
        rret, rcount = r[name]
        assert rcount == count, (name, count, rcount)
        want = {"npa_status": "npa_status", "void": "", "const char*": "*const c_char",
                "int": "c_int", "uint32_t": "u32", "size_t": "usize"}.get(ret.replace(" *", "*"), None)
        assert want is not None, (name, ret)
        assert rret == want, (name, ret, rret)


def test_every_struct_matches_field_order():
    h, r = header_structs(), rust_structs()
    assert h, "no structs parsed"
    for name, fields in h.items():
        assert name in r, name
        assert r[name] == fields, (name, fields, r[name])
    for opaque in ("npa_context", "npa_state", "npa_manifest"):
        assert opaque in r


def test_every_constant_has_the_header_value():
    h, r = header_constants(), rust_constants()
    assert len(h) >= 40
    for name, val in h.items():
        assert name in r, name
        assert r[name] == val, (name, val, r[name])


def _safe_methods():
    """Method name -> body text of each `pub fn` in the safe crate's impl blocks (the first one of a
    name: `Context::step` comes before `State::step`)."""
    text = open(SAFE).read()
    out = {}
    starts = [(m.group(1), m.start()) for m in re.finditer(r"\n    pub fn (\w+)", text)]
    for i, (name, at) in enumerate(starts):
        end = starts[i + 1][1] if i + 1 < len(starts) else len(text)
        out.setdefault(name, text[at:end])
    return out


def _sys_calls(body):
    """(sys function, argument count) of every `sys::npa_*(...)` call in a method body."""
    calls = []
    for m in re.finditer(r"sys::(npa_\w+)\(", body):
        depth, i, args, cur = 1, m.end(), [], ""
        while depth:
            c = body[i]
            if c in "([{":
                depth += 1
            elif c in ")]}":
                depth -= 1
            if depth == 1 and c == ",":
                args.append(cur)
                cur = ""
            elif depth:
                cur += c
            i += 1
        if cur.strip():
            args.append(cur)
        calls.append((m.group(1), len(args)))
    return calls


def test_safe_crate_wraps_the_reference_operators():
    methods = _safe_methods()
    sys_fns = rust_functions()
    want = {"build_hashgrid": "npa_build_hashgrid", "perceive_with_options": "npa_perceive",
            "euler_step": "npa_euler_step", "decode_gaussians_3d": "npa_decode_gaussians_3d",
            "splat_particles_2d": "npa_splat_2d", "step": "npa_step"}
    for method, fn in want.items():
        assert method in methods, method
        calls = dict(_sys_calls(methods[method]))
        assert fn in calls, (method, fn, calls)
        assert calls[fn] == sys_fns[fn][1], (method, fn, calls[fn], sys_fns[fn][1])
    for st in ("PerceptionOutput", "Gaussian3d", "HashGridSnapshot", "StepOutput"):
        assert re.search(r"pub struct %s\b" % st, open(SAFE).read()), st
