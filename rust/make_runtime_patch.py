"""Writes rust/patches/spissa-runtime-hip.patch: the changes to the Spissa
workspace that put the spissa-hip crate behind a `hip` cargo feature of
crates/spissa-runtime.

Every change is an insertion, so the default (CPU) build of the runtime is
unchanged and the patch carries one line of the workspace's own text around
each hunk:

- Cargo.toml: crates/spissa-hip joins the workspace members;
- crates/spissa-runtime/Cargo.toml: the optional dependency and the feature;
- crates/spissa-runtime/src/lib.rs: the hip_cache module (feature `hip`), and
  dead-code tolerance for rotary.rs under the feature;
- crates/spissa-runtime/src/rotary.rs: the CPU KvCache (rotary.rs:195-318) and
  the CPU attention (rotary.rs:335-415) with their private helpers
  (rotary.rs:483-599) are compiled without the feature; with it, KvCache is
  hip_cache::KvCache and the attention call forwards to the device;
- crates/spissa-runtime/src/hip_cache.rs: new, from
  rust/spissa-runtime/src/hip_cache.rs of this repository.

The crate itself is rust/spissa-hip of this repository, linked into the
workspace as crates/spissa-hip (a symlink: its build.rs finds the HIP sources
through its real location). The rollback of models/llama/session/mod.rs:745-771
needs no change: it calls KvCache::len and KvCache::truncate, which keep their
signatures; hip_cache.rs tests that sequence on device caches.

Usage: python rust/make_runtime_patch.py [--reference DIR] [--check]
(--check compares with the committed patch instead of writing it).
"""
from __future__ import annotations

import argparse
import difflib
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
PATCH = HERE / "patches" / "spissa-runtime-hip.patch"
NEW_FILES = {"crates/spissa-runtime/src/hip_cache.rs": HERE / "spissa-runtime" / "src" / "hip_cache.rs"}

NOT_HIP = '#[cfg(not(feature = "hip"))]'
HIP_SDPA = [
    "/// With the `hip` feature: the same call on the MI355X over the device cache",
    "/// (hip_cache.rs): split-K f32 decode for query_len == 1, bf16-MFMA flash",
    "/// prefill for longer chunks at head_dim 64, 128 and 256.",
    '#[cfg(feature = "hip")]',
    "pub fn scaled_dot_product_attention_with_cache(",
    "    q: &[f32],",
    "    current_k: &[f32],",
    "    current_v: &[f32],",
    "    cache: Option<&KvCache>,",
    "    config: KvAttentionConfig,",
    ") -> Result<Vec<f32>> {",
    "    crate::hip_cache::attention(q, current_k, current_v, cache, config)",
    "}",
    "",
]

# (file, [(anchor line, offset from the anchor, lines inserted there)]):
# the lines go before line index(anchor) + offset of the original file.
EDITS = [
    ("Cargo.toml", [
        ('    "crates/spissa-runtime",', 1, ['    "crates/spissa-hip",']),
    ]),
    ("crates/spissa-runtime/Cargo.toml", [
        ("log = { workspace = true }", 1, [
            'spissa-hip = { path = "../spissa-hip", optional = true }',
            "",
            "[features]",
            "# Device-resident KV cache and attention on AMD Instinct MI355X (gfx950)",
            "# through the spissa-hip crate; the default build is unchanged.",
            'hip = ["dep:spissa-hip"]',
        ]),
    ]),
    ("crates/spissa-runtime/src/lib.rs", [
        ("mod rotary;", 0, ['#[cfg_attr(feature = "hip", allow(dead_code))]']),
        ("mod rotary;", 1, ['#[cfg(feature = "hip")]', "mod hip_cache;"]),
    ]),
    ("crates/spissa-runtime/src/rotary.rs", [
        ("pub struct KvCache {", -1, [NOT_HIP]),
        ("impl KvCache {", 0, [NOT_HIP]),
        ("pub struct KvAttentionConfig {", -1, [
            "/// With the `hip` feature the cache is resident in HBM (hip_cache.rs): the",
            "/// same API, backed by the spissa-hip crate.",
            '#[cfg(feature = "hip")]',
            "pub use crate::hip_cache::KvCache;",
            "",
        ]),
        ("pub fn scaled_dot_product_attention_with_cache(", 0, [NOT_HIP]),
        ("fn validate_rotary_inputs(q: &[f32], k: &[f32], config: RotaryEmbeddingConfig) -> Result<()> {", 0,
         HIP_SDPA),
        ("fn validate_kv_attention_inputs(", 0, [NOT_HIP]),
        ("fn softmax_inplace(logits: &mut [f32]) -> Result<()> {", 0, [NOT_HIP]),
        ("enum KvTensorKind {", -1, [NOT_HIP]),
        ("fn kv_row<'a>(", 0, [NOT_HIP]),
    ]),
]


def edited(lines: list[str], edits) -> list[str]:
    inserts: dict[int, list[str]] = {}
    for anchor, offset, add in edits:
        hits = [i for i, line in enumerate(lines) if line == anchor]
        if len(hits) != 1:
            raise SystemExit(f"anchor {anchor!r} found {len(hits)} times")
        inserts.setdefault(hits[0] + offset, []).extend(add)
    out = []
    for i, line in enumerate(lines):
        out.extend(inserts.pop(i, []))
        out.append(line)
    out.extend(inserts.pop(len(lines), []))
    if inserts:
        raise SystemExit(f"insert positions outside the file: {sorted(inserts)}")
    return out


def make_patch(reference: Path) -> str:
    chunks = []
    for rel, edits in EDITS:
        old = (reference / rel).read_text().splitlines()
        new = edited(old, edits)
        diff = difflib.unified_diff(old, new, f"a/{rel}", f"b/{rel}", n=1, lineterm="")
        chunks.append("\n".join(diff) + "\n")
    for rel, src in NEW_FILES.items():
        new = src.read_text().splitlines()
        diff = difflib.unified_diff([], new, "/dev/null", f"b/{rel}", n=0, lineterm="")
        chunks.append("\n".join(diff) + "\n")
    return "".join(chunks)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    ap.add_argument("--check", action="store_true")
    args = ap.parse_args()
    text = make_patch(Path(args.reference))
    if args.check:
        same = PATCH.read_text() == text
        print("up to date" if same else "stale: regenerate with python rust/make_runtime_patch.py")
        return 0 if same else 1
    PATCH.parent.mkdir(exist_ok=True)
    PATCH.write_text(text)
    print(PATCH)
    return 0


if __name__ == "__main__":
    sys.exit(main())
