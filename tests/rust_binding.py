"""Reads the C ABI declarations of include/g4attn.h and the Rust crate's
`extern "C"` block, and maps C parameter types to the Rust types a binding
must use.  No Rust toolchain is needed: the checks are textual, on the
declarations themselves.
"""
import re

RUST_KEYWORDS = {
    "as", "break", "const", "continue", "crate", "else", "enum", "extern", "false", "fn", "for", "if", "impl",
    "in", "let", "loop", "match", "mod", "move", "mut", "pub", "ref", "return", "self", "Self", "static",
    "struct", "super", "trait", "true", "type", "unsafe", "use", "where", "while", "async", "await", "dyn",
    "abstract", "become", "box", "do", "final", "macro", "override", "priv", "typeof", "unsized", "virtual",
    "yield", "try",
}

# C scalar / opaque names -> Rust names (std::ffi for the C ones).
BASE = {
    "int": "c_int", "char": "c_char", "void": "c_void", "float": "f32", "double": "f64", "size_t": "usize",
    "int8_t": "i8", "uint8_t": "u8", "uint16_t": "u16", "int32_t": "i32", "int64_t": "i64",
    "uint64_t": "u64", "g4_ctx": "G4Ctx", "g4_kv_cache": "G4KvCache", "g4_hparams": "G4Hparams",
}


def strip_c_comments(text):
    text = re.sub(r"/\*.*?\*/", " ", text, flags=re.S)
    return re.sub(r"//[^\n]*", " ", text)


def strip_rust_comments(text):
    return re.sub(r"//[^\n]*", " ", text)


def c_to_rust(ctype):
    """'const float **' -> '*mut *const f32'; 'g4_stream' -> '*mut c_void';
    'void' (a return type) -> '()'."""
    t = " ".join(ctype.replace("*", " * ").split())
    stars = t.count("*")
    words = [w for w in t.split() if w != "*"]
    const = "const" in words
    words = [w for w in words if w not in ("const", "struct", "enum")]
    assert len(words) == 1, ctype
    base = words[0]
    if base == "g4_stream":  # typedef void *g4_stream
        assert stars == 0, ctype
        return "*mut c_void"
    if base == "g4_status":
        assert stars == 0, ctype
        return "c_int"
    rust = BASE[base]
    if stars == 0:
        return "()" if base == "void" else rust
    out = ("*const " if const else "*mut ") + rust
    for _ in range(stars - 1):
        out = "*mut " + out
    return out


def parse_header(path):
    """[(name, return C type, [(param C type, param name), ...])] for every
    function the header declares, in order."""
    text = strip_c_comments(open(path).read())
    text = re.sub(r"typedef\s+(struct|enum)\s*\w*\s*\{.*?\}\s*\w+\s*;", " ", text, flags=re.S)
    text = re.sub(r"#[^\n]*", " ", text)
    text = text.replace('extern "C" {', " ")
    out = []
    for m in re.finditer(r"([A-Za-z_][\w\s\*]*?)\b(g4_\w+)\s*\(([^;{}]*?)\)\s*;", text):
        ret, name, params = " ".join(m.group(1).split()), m.group(2), " ".join(m.group(3).split())
        if ret.startswith("typedef"):
            continue
        plist = []
        if params and params != "void":
            for p in params.split(","):
                p = p.strip()
                pm = re.match(r"(.*?)(\w+)$", p)
                plist.append((pm.group(1).strip(), pm.group(2)))
        out.append((name, ret, plist))
    return out


def parse_header_struct(path, name):
    """[(C type, field)] of `typedef struct { ... } name;`."""
    text = strip_c_comments(open(path).read())
    m = re.search(r"typedef\s+struct\s*\{(.*?)\}\s*" + name + r"\s*;", text, flags=re.S)
    fields = []
    for decl in m.group(1).split(";"):
        decl = " ".join(decl.split())
        if not decl:
            continue
        ctype, names = decl.split(" ", 1)
        fields += [(ctype, n.strip()) for n in names.split(",")]
    return fields


def parse_header_enum(path):
    text = strip_c_comments(open(path).read())
    return {k: int(v) for k, v in re.findall(r"\b(G4_\w+)\s*=\s*(\d+)", text)}


def parse_rust_externs(path):
    """{name: (return Rust type, [(param, Rust type)])} of the `fn`
    declarations inside the file's `extern "C"` blocks."""
    text = strip_rust_comments(open(path).read())
    out = {}
    for block in re.finditer(r'extern\s+"C"\s*\{(.*?)\n\}', text, flags=re.S):
        for m in re.finditer(r"(?:pub\s+)?fn\s+(\w+)\s*\((.*?)\)\s*(?:->\s*([^;]+?))?\s*;", block.group(1),
                             flags=re.S):
            name, params, ret = m.group(1), " ".join(m.group(2).split()), (m.group(3) or "()").strip()
            plist = []
            for p in [p for p in params.split(",") if p.strip()]:
                pname, ptype = p.split(":", 1)
                plist.append((pname.strip(), " ".join(ptype.split())))
            out[name] = (" ".join(ret.split()), plist)
    return out


def rust_calls(text, prefix="ffi::"):
    """[(function, argument count)] of every `ffi::name(...)` call in Rust
    source text, counting top-level commas inside balanced brackets."""
    text = strip_rust_comments(text)
    calls = []
    for m in re.finditer(re.escape(prefix) + r"(\w+)\s*\(", text):
        i, depth, args, cur = m.end(), 1, [], ""
        while depth:
            c = text[i]
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
