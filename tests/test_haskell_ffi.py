"""The Haskell drop-in (haskell/) against the C ABI, on the CPU.

There is no GHC in this image, so the modules under haskell/ are not
compiled here.  What can be checked without it is the FFI boundary: every
`foreign import ccall` of haskell/Graphics/HIP.hs must name a function that
include/gemma_hip.h declares, with the same arity and, argument by
argument, the Haskell type that marshals the C type; finaliser imports
(`&name` as FinalizerPtr) must name void functions of one handle pointer.
The rewired modules may call only imports that exist, and the exports of
Gemma.Model / Gemma.Layers.LinearQ4 keep the reference's names
(src/Gemma/Model.hs:19-31, src/Gemma/Layers/LinearQ4.hs:17-21).
"""
from __future__ import annotations

import re
from pathlib import Path

import pytest

from conftest import REPO

HS = REPO / "haskell"
HEADER = REPO / "include" / "gemma_hip.h"

SCALARS = {"int": "CInt", "int32_t": "Int32", "int64_t": "Int64", "uint64_t": "Word64", "uint32_t": "Word32",
           "size_t": "CSize", "float": "CFloat", "double": "CDouble"}
POINTEES = {"float": "CFloat", "double": "CDouble", "int32_t": "Int32", "uint8_t": "Word8", "uint32_t": "Word32",
            "gh_ctx": "CtxS", "gh_model": "ModelS", "gh_kv": "KvS", "gh_q4": "Q4S", "gh_config": "GhConfig",
            "int": "CInt", "size_t": "CSize"}


def c_prototypes() -> dict[str, tuple[str, list[str]]]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for ret, name, args in re.findall(r"([A-Za-z_][\w \*]*?)\s*\b(gh_\w+)\s*\(([^)]*)\)\s*;", text):
        args = [a.strip() for a in args.split(",")] if args.strip() not in ("", "void") else []
        out[name] = (ret.strip(), args)
    return out


def c_to_hs(ctype: str) -> str:
    """The Haskell FFI type that marshals a C parameter type."""
    t = re.sub(r"\bconst\b", "", ctype)
    t = re.sub(r"\s+[A-Za-z_]\w*$", "", t.strip())  # drop the parameter name
    stars = t.count("*")
    base = t.replace("*", "").strip()
    if stars == 0:
        return SCALARS[base]
    if base == "char" and stars == 1:
        return "CString"
    if base == "void" and stars == 1:
        return "Ptr *"  # any pointee
    inner = POINTEES[base]
    for _ in range(stars):
        inner = f"Ptr ({inner})" if " " in inner else f"Ptr {inner}"
    return inner


def hs_imports() -> list[tuple[str, str, str]]:
    """(C name incl. a leading '&' for address imports, Haskell name, type)."""
    text = (HS / "Graphics" / "HIP.hs").read_text()
    pat = re.compile(r'foreign import ccall (?:safe |unsafe )?"(&?\w+)"\s+(\w+)\s*::\s*(.*?)(?=\nforeign import|\n\n|\n--)',
                     re.S)
    return [(c, h, " ".join(t.split())) for c, h, t in pat.findall(text)]


def split_arrows(t: str) -> list[str]:
    parts, depth, cur = [], 0, ""
    i = 0
    while i < len(t):
        ch = t[i]
        if ch == "(":
            depth += 1
        elif ch == ")":
            depth -= 1
        if depth == 0 and t.startswith("->", i):
            parts.append(cur.strip())
            cur = ""
            i += 2
            continue
        cur += ch
        i += 1
    parts.append(cur.strip())
    return parts


def norm(t: str) -> str:
    t = " ".join(t.split())
    while t.startswith("(") and t.endswith(")"):
        t = t[1:-1].strip()
    return t


def test_every_foreign_import_matches_the_header():
    protos = c_prototypes()
    imports = hs_imports()
    assert len(imports) == len(re.findall(r"^foreign import", (HS / "Graphics" / "HIP.hs").read_text(), re.M)) >= 30
    for cname, hname, htype in imports:
        addr = cname.startswith("&")
        name = cname.lstrip("&")
        assert name in protos, f"{hname}: {name} is not declared in include/gemma_hip.h"
        ret, args = protos[name]
        if addr:
            # a finaliser: void f(T*), imported as FinalizerPtr T
            assert ret == "void" and len(args) == 1, (name, ret, args)
            m = re.fullmatch(r"FinalizerPtr (\w+)", htype)
            assert m, (hname, htype)
            assert c_to_hs(args[0]) == f"Ptr {m.group(1)}", (name, args[0], htype)
            continue
        parts = [norm(p) for p in split_arrows(htype)]
        *hargs, hret = parts
        assert len(hargs) == len(args), f"{hname}: arity {len(hargs)} != {len(args)} of {name}{tuple(args)}"
        for i, (ca, ha) in enumerate(zip(args, hargs)):
            want = c_to_hs(ca)
            if want == "Ptr *":
                assert re.fullmatch(r"Ptr (\(\)|\w+)", ha), (hname, i, ca, ha)
            else:
                assert ha == want, f"{hname} argument {i}: C '{ca}' wants {want}, Haskell has {ha}"
        want_ret = {"int": "IO CInt", "const char*": "IO CString", "void": "IO ()"}[ret.replace(" *", "*")]
        assert hret == want_ret, (hname, ret, hret)


def test_config_storable_matches_gh_config():
    """GhConfig's Storable instance covers gh_config's 15 four-byte fields in
    order (the ctypes mirror gives the C layout)."""
    import ctypes as C
    from gemma_hip._lib import GhConfig
    text = (HS / "Graphics" / "HIP.hs").read_text()
    assert "sizeOf _ = 15 * 4" in text and C.sizeof(GhConfig) == 60
    names = [n for n, _ in GhConfig._fields_]
    assert names[:7] == ["vocab", "hidden", "n_layers", "n_heads", "n_kv_heads", "head_dim", "ffn"]
    offsets = {n: getattr(GhConfig, n).offset for n in names}
    for field, off in (("ghThetaLocal", "rope_theta_local"), ("ghThetaGlobal", "rope_theta_global"),
                       ("ghRmsEps", "rms_eps"), ("ghMode", "mode"), ("ghFlags", "flags")):
        assert f"pokeByteOff p {offsets[off]} ({field} c)" in text, (field, offsets[off])


def test_rewired_modules_use_only_existing_imports_and_keep_the_reference_exports():
    imported = {h for _, h, _ in hs_imports()}
    for path in (HS / "Gemma" / "Model.hs", HS / "Gemma" / "Layers" / "LinearQ4.hs"):
        text = path.read_text()
        for used in set(re.findall(r"HIP\.(c_\w+|p_\w+)", text)):
            assert used in imported, (path.name, used)
    model = (HS / "Gemma" / "Model.hs").read_text()
    exports = re.search(r"module Gemma\.Model\s*\((.*?)\)\s*where", model, re.S).group(1)
    for name in ("GemmaConfig(..)", "GemmaModel(..)", "gemma3_1BConfig", "loadGemmaModel", "loadGemmaModelFromGGUF",
                 "configFromGGUF", "runGemmaInference", "runGemmaInferenceCached",
                 "runGemmaInferenceCachedWithLayer0"):
        assert name in exports, name
    for sig in ("runGemmaInferenceCached :: GemmaModel dtype\n                        -> Vector Int\n"
                "                        -> Maybe KVCache\n                        -> IO (Vector Float, KVCache)",
                "loadGemmaModelFromGGUF :: FilePath -> ContT r IO (GemmaModel dtype)",
                "loadGemmaModel :: FilePath -> GemmaConfig -> IO (GemmaModel dtype)"):
        assert sig in model, sig
    lq = (HS / "Gemma" / "Layers" / "LinearQ4.hs").read_text()
    for name in ("runLinearQ4", "runLinearQ4WithContext", "runLinearQ4GPU"):
        assert re.search(rf"^{name} ::", lq, re.M), name


@pytest.mark.parametrize("planted", ["arity", "type", "name", "finaliser"])
def test_signature_check_catches_planted_mismatches(planted, monkeypatch):
    """The checker itself fails on a wrong import: a dropped argument, a
    wrong argument type, an undeclared name, an int-returning finaliser."""
    good = hs_imports()
    bad = list(good)
    i = next(k for k, (c, _, _) in enumerate(good) if c == "gh_step")
    c, h, t = bad[i]
    if planted == "arity":
        bad[i] = (c, h, t.replace("Int32 -> ", "", 1))
    elif planted == "type":
        bad[i] = (c, h, t.replace("Int32", "CInt", 1))
    elif planted == "name":
        bad[i] = ("gh_stepp", h, t)
    else:
        bad.append(("&gh_kv_destroy", "p_bad", "FinalizerPtr KvS"))
    monkeypatch.setattr(__import__(__name__), "hs_imports", lambda: bad)
    with pytest.raises(AssertionError):
        test_every_foreign_import_matches_the_header()


# ---------------------------------------------------------------- imports
# The reference library's build-depends (gemma.cabal:58-71) without
# webgpu-dawn, which Graphics.HIP replaces.
REFERENCE_DEPENDS = {"base", "vector", "bytestring", "aeson", "text", "containers", "transformers", "mtl", "half",
                     "directory", "process", "filepath"}
# Package modules the drop-in imports, by the package that provides them.
PACKAGE_MODULES = {
    "base": {"Control.Exception", "Control.Monad", "Control.Monad.IO.Class", "Data.Bits", "Data.Int", "Data.Maybe",
             "Data.Word", "Foreign.C.String", "Foreign.C.Types", "Foreign.ForeignPtr", "Foreign.Marshal.Alloc",
             "Foreign.Ptr", "Foreign.Storable"},
    "vector": {"Data.Vector", "Data.Vector.Storable", "Data.Vector.Storable.Mutable"},
    "text": {"Data.Text"},
    "transformers": {"Control.Monad.Trans.Cont"},
}
# Modules of the reference library (gemma.cabal exposed-modules) the drop-in
# imports, with the names it takes from each (constructors under their type).
REFERENCE_MODULES = {
    "Gemma.KVCache": {"KVCache", "LayerKVCache", "cacheLength", "initKVCache"},
    "Gemma.SafeTensors": {"getTensor", "hasTensor", "loadSafeTensors"},
    "Gemma.GGUF": {"GGUFFile", "MetadataValue", "MetaArray", "getMetadata", "getMetadataInt", "getMetadataFloat",
                   "getTensorShape", "hasTensor"},
}
REFERENCE = Path("/root/reference")


def hs_module_imports(text: str) -> list[tuple[str, set[str]]]:
    """(module, names used from it) for every import of a module's text: the
    explicit import list, or the Alias.name uses of a qualified import."""
    out = []
    for m in re.finditer(r"^import\s+(qualified\s+)?([A-Z][\w.]*)(?:\s+as\s+(\w+))?\s*(\(([^()]*(?:\([^()]*\)[^()]*)*)\))?",
                         text, re.M):
        qual, mod, alias, _, items = m.groups()
        names = set()
        if items is not None:
            for it in items.split(","):
                it = it.strip()
                if it:
                    names.add(re.sub(r"\(.*\)$", "", it).strip())
        if alias:
            names |= set(re.findall(rf"\b{re.escape(alias)}\.([A-Za-z_]\w*)", text))
        out.append((mod, names))
    return out


def committed_modules() -> dict[str, Path]:
    return {".".join(p.relative_to(HS).with_suffix("").parts): p for p in HS.rglob("*.hs")}


def exports_of(text: str, mod: str) -> str:
    m = re.search(rf"module\s+{re.escape(mod)}\s*\((.*?)\)\s*where", text, re.S)
    assert m, mod
    return m.group(1)


def exported_names(text: str, mod: str) -> set[str]:
    """Names a module exports: its export list, plus the constructors and
    record fields of every type exported with (..)."""
    exp = exports_of(text, mod)
    names = set(re.findall(r"[A-Za-z_][\w']*", exp))
    for t in re.findall(r"\b([A-Z]\w*)\(\.\.\)", exp):
        m = re.search(rf"^data {t}\b(.*?)(?=^\S)", text, re.S | re.M)
        if m:
            names |= set(re.findall(r"[A-Za-z_][\w']*", m.group(1)))
    return names


def unresolved_imports(files: dict[str, str]) -> list[str]:
    """Every import of the given module texts that does not resolve."""
    bad = []
    mods = committed_modules()
    for path, text in files.items():
        for mod, names in hs_module_imports(text):
            if mod in mods:
                exp = exported_names(mods[mod].read_text(), mod)
                bad += [f"{path}: {mod}.{n} not exported" for n in names if n not in exp and not n.startswith("(")]
            elif mod in REFERENCE_MODULES:
                bad += [f"{path}: {mod}.{n} not among the reference names" for n in names - REFERENCE_MODULES[mod]]
            elif not any(mod in ms and pkg in REFERENCE_DEPENDS for pkg, ms in PACKAGE_MODULES.items()):
                bad.append(f"{path}: module {mod} is neither committed, nor the reference's, nor a dependency's")
    return bad


def test_every_haskell_import_resolves():
    """Each import under haskell/ names a committed module (exporting what is
    imported), a module of the reference library, or a module of a package
    the reference already depends on: the module graph is complete."""
    files = {str(p.relative_to(HS)): p.read_text() for p in HS.rglob("*.hs")}
    assert len(files) >= 3
    assert unresolved_imports(files) == []


def test_reference_modules_export_the_names_the_drop_in_takes():
    """The reference-side names in REFERENCE_MODULES exist: each module is an
    exposed module of gemma.cabal and exports the name (or the type whose
    constructor it is).  Reads the reference tree as text; skipped where it
    is absent."""
    if not (REFERENCE / "gemma.cabal").exists():
        pytest.skip("reference tree not present")
    cabal = (REFERENCE / "gemma.cabal").read_text()
    exposed = re.search(r"exposed-modules:\s*(.*?)\n\s*\n|exposed-modules:\s*(.*?)hs-source-dirs", cabal, re.S)
    block = next(g for g in exposed.groups() if g)
    for mod, names in REFERENCE_MODULES.items():
        assert re.search(rf"^\s*{re.escape(mod)}\s*$", block, re.M), mod
        text = (REFERENCE / "src" / Path(*mod.split("."))).with_suffix(".hs").read_text()
        exp = exports_of(text, mod)
        for n in names:
            ok = re.search(rf"\b{re.escape(n)}\b", exp) or re.search(rf"[=|]\s*{re.escape(n)}\b", text)
            assert ok, (mod, n)
    deps = re.search(r"library.*?build-depends:(.*?)\n\s*\n", cabal, re.S).group(1)
    for pkg in REFERENCE_DEPENDS:
        assert re.search(rf"\b{re.escape(pkg)}\b", deps), pkg


def test_import_check_catches_a_missing_module():
    """A module the tree does not hold (the former Gemma.Model.Config) and a
    name a committed module does not export both fail the check."""
    text = (HS / "Gemma" / "Model.hs").read_text()
    planted = text.replace("import qualified Gemma.GGUF as GGUF",
                           "import qualified Gemma.GGUF as GGUF\nimport Gemma.Model.Config (GemmaConfig(..))")
    assert any("Gemma.Model.Config" in b for b in unresolved_imports({"Model.hs": planted}))
    planted = text.replace("import Graphics.HIP (check)", "import Graphics.HIP (check, c_noSuchCall)")
    assert any("c_noSuchCall" in b for b in unresolved_imports({"Model.hs": planted}))
