"""The Rust crate recipe in INTEGRATION.md against the build that this
repository runs (spissa_amd/build.py) and the C header.

No cargo exists in this image, so the recipe is never compiled here; these
checks keep it in step instead: the same flags for every source, the same
per-file additions, every csrc/*.hip source (by a directory listing, not a
fixed list), the same link line, and Rust extern declarations whose names and
parameter counts match include/spissa_hip.h.
"""
import re
from pathlib import Path

from spissa_amd import build

ROOT = Path(__file__).resolve().parent.parent
DOC = (ROOT / "INTEGRATION.md").read_text()


def rust_block(title: str) -> str:
    start = DOC.index(title)
    body = DOC[start:]
    m = re.search(r"```rust\n(.*?)```", body, flags=re.S)
    assert m, f"no rust block after {title}"
    return m.group(1)


BUILD_RS = rust_block("### `crates/spissa-hip/build.rs`")
LIB_RS = rust_block("### `crates/spissa-hip/src/lib.rs`")


def str_list(src: str, name: str):
    m = re.search(rf"const {name}: &\[&str\] = &\[(.*?)\];", src, flags=re.S)
    assert m, f"const {name} missing from build.rs"
    return re.findall(r'"([^"]*)"', m.group(1))


def test_common_flags_match_build_py():
    want = [f for f in build.COMMON if not f.startswith("-I")]
    assert str_list(BUILD_RS, "COMMON") == want
    # the include directory is passed as -I<root>/../include, as build.py's -I<repo>/include
    assert 'format!("-I{}", root.join("../include").display())' in BUILD_RS
    assert any(f.startswith("-I") and f.endswith("include") for f in build.COMMON)


def test_per_source_flags_match_build_py():
    m = re.search(r"const EXTRA: &\[\(&str, &\[&str\]\)\] = &\[(.*?)\n\];", BUILD_RS, flags=re.S)
    assert m
    extra = {}
    for name, flags in re.findall(r'\("([^"]+)",\s*&\[(.*?)\]\)', m.group(1), flags=re.S):
        extra[name] = re.findall(r'"([^"]*)"', flags)
    assert extra == build.EXTRA
    for name in extra:
        assert (build.CSRC / name).exists(), name


def test_sources_are_every_hip_file_of_csrc():
    # a directory listing filtered to .hip and sorted, as build.py globs
    assert 'fs::read_dir(root.join("csrc"))' in BUILD_RS
    assert 'x == "hip"' in BUILD_RS and "srcs.sort()" in BUILD_RS
    assert "let srcs = [" not in BUILD_RS  # no fixed list that could miss a file
    # what the recipe would compile is what build.py compiles
    assert sorted(p.name for p in build.CSRC.glob("*.hip")) == sorted(
        p.name for p in build.CSRC.iterdir() if p.suffix == ".hip")
    assert {"abi.hip", "linear.hip", "sampling.hip", "decode.hip", "prefill.hip"} <= {
        p.name for p in build.CSRC.glob("*.hip")}


def test_link_line_matches_build_py():
    assert str_list(BUILD_RS, "LINK") == build.LINK
    assert str_list(BUILD_RS, "LINK_LIBS") == build.LINK_LIBS
    assert "cmd = [HIPCC, *LINK, \"-o\", str(tmp), *map(str, objs), *LINK_LIBS]" in Path(
        build.__file__).read_text()
    assert build.ARCH == "gfx950"


def header_params():
    text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / "spissa_hip.h").read_text(), flags=re.S)
    out = {}
    for name, args in re.findall(r"\b(spissa_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        args = args.strip()
        out[name] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def test_rust_extern_declarations_match_the_header():
    hdr = header_params()
    decls = re.findall(r"pub fn (spissa_[a-z0-9_]+)\((.*?)\)", LIB_RS, flags=re.S)
    assert len(decls) >= 20
    for name, args in decls:
        assert name in hdr, f"{name} is not declared in spissa_hip.h"
        n = 0 if not args.strip() else args.count(":")
        assert n == hdr[name], f"{name}: {n} Rust parameters, {hdr[name]} in the header"
