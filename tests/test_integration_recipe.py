"""The Rust side of the boundary (rust/spissa-hip, rust/patches) against the
build this repository runs (spissa_amd/build.py), the C header and the
reference workspace.

No cargo exists in this image, so the crate is never compiled here; these
checks keep it in step instead:
- build.rs: the same flags for every source, the same per-file additions,
  every csrc/*.hip source (by a directory listing, not a fixed list), the
  same link line;
- src/lib.rs: one `extern "C"` declaration per function of
  include/spissa_hip.h, with the same name and parameter count, and repr(C)
  structs with the header's fields in order;
- the runtime patch: regenerated from its script it is byte-identical to the
  committed file, and it applies to the reference workspace (patch --dry-run
  there, which writes nothing, and a real application to a scratch copy of
  the touched files).
"""
import re
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

from spissa_amd import build

ROOT = Path(__file__).resolve().parent.parent
CRATE = ROOT / "rust" / "spissa-hip"
BUILD_RS = (CRATE / "build.rs").read_text()
LIB_RS = (CRATE / "src" / "lib.rs").read_text()
HEADER = (ROOT / "include" / "spissa_hip.h").read_text()
PATCH = ROOT / "rust" / "patches" / "spissa-runtime-hip.patch"
REFERENCE = Path("/root/reference")

sys.path.insert(0, str(ROOT / "rust"))
import make_runtime_patch  # noqa: E402


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
    # the default source root is ../../spissa_amd from the crate's real location
    assert (CRATE / "../../spissa_amd").resolve() == build.PKG


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
    assert {"abi.hip", "linear.hip", "sampling.hip", "decode.hip", "prefill.hip"} <= {
        p.name for p in build.CSRC.glob("*.hip")}


def test_link_line_matches_build_py():
    assert str_list(BUILD_RS, "LINK") == build.LINK
    assert str_list(BUILD_RS, "LINK_LIBS") == build.LINK_LIBS
    assert "cmd = [HIPCC, *LINK, \"-o\", str(tmp), *map(str, objs), *LINK_LIBS]" in Path(
        build.__file__).read_text()
    assert build.ARCH == "gfx950"


def header_params():
    text = re.sub(r"/\*.*?\*/", "", HEADER, flags=re.S)
    out = {}
    for name, args in re.findall(r"\b(spissa_[a-z0-9_]+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        args = args.strip()
        out[name] = 0 if args in ("", "void") else args.count(",") + 1
    return out


def rust_decls():
    block = LIB_RS[LIB_RS.index('extern "C" {'):]
    return {name: (0 if not args.strip() else args.count(":"))
            for name, args in re.findall(r"pub fn (spissa_[a-z0-9_]+)\((.*?)\)", block, flags=re.S)}


def test_every_header_function_is_declared_in_the_crate():
    hdr, rs = header_params(), rust_decls()
    assert len(hdr) >= 50
    assert set(hdr) == set(rs), (sorted(set(hdr) - set(rs)), sorted(set(rs) - set(hdr)))
    for name, n in hdr.items():
        assert rs[name] == n, f"{name}: {rs[name]} Rust parameters, {n} in the header"


def c_struct_fields(name: str):
    m = re.search(r"typedef struct \{([^{}]*)\}\s*" + name + ";", HEADER)
    assert m, name
    body = re.sub(r"/\*.*?\*/", "", m.group(1), flags=re.S)
    return [re.findall(r"(\w+)\s*;", line)[0] for line in body.splitlines() if ";" in line]


def rust_struct_fields(name: str):
    m = re.search(r"pub struct " + name + r" \{(.*?)\n    \}", LIB_RS, flags=re.S)
    assert m, name
    return re.findall(r"pub (\w+):", m.group(1))


@pytest.mark.parametrize("name", ["spissa_rotary_config", "spissa_kv_attention_config", "spissa_attention_plan",
                                  "spissa_linear_config", "spissa_attention_layer"])
def test_repr_c_structs_follow_the_header(name):
    assert rust_struct_fields(name) == c_struct_fields(name)
    assert f"#[repr(C)]" in LIB_RS.split(f"pub struct {name}")[0][-80:]


def test_status_codes_follow_the_header():
    for code, value in re.findall(r"(SPISSA_ERR_\w+|SPISSA_OK) = (\d+)", HEADER):
        assert re.search(rf"pub const {code}: c_int = {value};", LIB_RS), code


def test_runtime_patch_is_generated_from_this_repository():
    if not REFERENCE.is_dir():
        pytest.skip("the reference workspace is not on this machine")
    assert make_runtime_patch.make_patch(REFERENCE) == PATCH.read_text()


def test_runtime_patch_applies_to_the_reference_workspace(tmp_path):
    if not REFERENCE.is_dir():
        pytest.skip("the reference workspace is not on this machine")
    if shutil.which("patch") is None:
        pytest.skip("no patch tool")
    # --dry-run on the workspace itself writes nothing
    res = subprocess.run(["patch", "-p1", "--dry-run", "-d", str(REFERENCE), "-i", str(PATCH)],
                         capture_output=True, text=True)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "FAILED" not in res.stdout and "offset" not in res.stdout and "fuzz" not in res.stdout
    # a real application to a copy of the touched files
    touched = [rel for rel, _ in make_runtime_patch.EDITS]
    for rel in touched:
        dst = tmp_path / rel
        dst.parent.mkdir(parents=True, exist_ok=True)
        shutil.copyfile(REFERENCE / rel, dst)
    res = subprocess.run(["patch", "-p1", "-d", str(tmp_path), "-i", str(PATCH)], capture_output=True, text=True)
    assert res.returncode == 0, res.stdout + res.stderr
    rotary = (tmp_path / "crates/spissa-runtime/src/rotary.rs").read_text()
    # every CPU-only item of the cache and the attention is gated, and the
    # feature brings in the device versions
    for item in ("pub struct KvCache {", "impl KvCache {", "fn validate_kv_attention_inputs(",
                 "fn softmax_inplace(", "enum KvTensorKind {", "fn kv_row<'a>("):
        before = rotary[:rotary.index(item)].rstrip().splitlines()
        assert '#[cfg(not(feature = "hip"))]' in before[-2:], item
    assert rotary.count("pub fn scaled_dot_product_attention_with_cache(") == 2
    assert 'pub use crate::hip_cache::KvCache;' in rotary
    hip = (tmp_path / "crates/spissa-runtime/src/hip_cache.rs").read_text()
    assert hip == (ROOT / "rust/spissa-runtime/src/hip_cache.rs").read_text()
    manifest = (tmp_path / "crates/spissa-runtime/Cargo.toml").read_text()
    assert 'hip = ["dep:spissa-hip"]' in manifest
    assert '"crates/spissa-hip"' in (tmp_path / "Cargo.toml").read_text()


def test_the_patched_runtime_uses_only_what_the_crate_exports():
    hip = (ROOT / "rust/spissa-runtime/src/hip_cache.rs").read_text()
    used = set(re.findall(r"spissa_hip::\{([^}]*)\}", hip)[0].replace(" ", "").split(","))
    used |= set(re.findall(r"spissa_hip::(\w+)\(", hip))
    exported = set(re.findall(r"pub (?:struct|enum|fn|type) (\w+)", LIB_RS)) | {"AttnConfigC"}
    assert used <= exported, used - exported
    # the methods the runtime calls on DeviceKvCache exist (clone: its Clone impl)
    assert "impl Clone for DeviceKvCache" in LIB_RS
    for method in set(re.findall(r"self\.device\.(\w+)\(", hip)) - {"clone"}:
        assert re.search(rf"pub fn {method}\(", LIB_RS), method
