"""CPU checks of the host launch arithmetic (spissa_plan_attention) against the
kernels' own index ranges, with no GPU.

For every plan the library reports, this replays what each workgroup of the
kernel would read and write, using the range formulas of decode_split_kernel
and decode_combine_kernel (decode.hip) and prefill_kernel (prefill.hip), and
checks that
  - the splits of every (sequence, head) cover exactly the keys its queries
    may see (rotary.rs:355,362-365 causal mask, plus the window), once each;
  - every partial a split writes, and every staged row the prefill reads, lies
    inside the workspace the plan sizes.
Shapes: every BASELINE config, the windowed non-causal chunks that once
dropped key tiles, and a seeded sweep.
"""
import random

import pytest

from spissa_amd import _ffi
from spissa_amd.device import plan_attention
from spissa_amd.errors import ShapeError
from spissa_amd.rotary import KvAttentionConfig

MAX_DECODE_BATCH = 16
MAX_DECODE_SPLITS = 512
SCRATCH_BYTES = 8 << 20
TILE_ALIGN = 64


def check_decode(cfg, past, plan, noalloc=False):
    """decode_split_kernel: grid (Hkv*HB, max_splits, B); split s of sequence b
    covers cached keys [kstart + s*kps, min(P, kstart + (s+1)*kps)) where
    kstart = max(0, P + 1 - W) with a window, for s < ceil((P - kstart) / kps);
    with token_split the new token (key P) is split 0 of its own (dispatched
    first) and cached split s is grid split s + 1, else cached split 0 takes
    it (one split at least)."""
    D, Hq, Hkv, W = cfg.head_dim, cfg.num_heads, cfg.kv_heads, cfg.window
    assert plan["path"] == _ffi.KERNEL_DECODE
    RB, HB, kps = plan["heads_per_block"], plan["head_blocks"], plan["keys_per_split"]
    assert RB * HB == Hq // Hkv and kps > 0
    entry = RB * (D + 2)
    B = min(len(past), MAX_DECODE_BATCH)  # the plan describes the first launch
    max_splits = plan["splits"]
    assert max_splits <= MAX_DECODE_SPLITS
    assert max_splits >= 1
    assert plan["workgroups"] == B * Hkv * HB * max_splits
    groups = B * Hkv * HB
    assert plan["partial_bytes"] >= groups * max_splits * entry * 4
    if noalloc:
        assert plan["partial_bytes"] <= SCRATCH_BYTES
    for b in range(B):
        P = past[b]
        kstart = max(0, P + 1 - W) if W > 0 else 0
        ncached = -(-(P - kstart) // kps)
        nsplit = ncached + 1 if plan["token_split"] else max(1, ncached)
        assert nsplit <= max_splits
        covered = []
        for s in range(nsplit):
            cs = s - 1 if plan["token_split"] else s
            if cs < 0:
                continue  # the token's own split reads no cached row
            k0 = kstart + cs * kps
            k1 = min(P, k0 + kps)
            assert k0 < k1 or (cs == 0 and P == kstart)  # cached split 0 holds at least the new token
            covered.append((k0, k1))
            for h in range(Hkv):
                for hb in range(HB):
                    bhh = (b * Hkv + h) * HB + hb
                    end = ((bhh * max_splits + s) + 1) * entry  # floats written by this split
                    assert end * 4 <= plan["partial_bytes"]
        # contiguous, disjoint, exactly [kstart, P), and key P in split 0
        pos = kstart
        for k0, k1 in covered:
            assert k0 == pos
            pos = k1
        assert pos == P


def check_prefill_grid(plan, n_qblocks, Hkv, HB, splits):
    """prefill_kernel's workgroup id -> (KV head, head block, split, query
    block) decode: every tuple exactly once; with xcd_group 1, the workgroups
    of one (KV head, split) have ids equal mod 8 (one XCD) and the padding ids
    decode to units past the last; with xcd_group 2, each XCD's ids take a
    contiguous run of the unsplit order (query blocks adjacent) and the
    padding ids decode past its end."""
    G = HB * n_qblocks
    units = Hkv * splits
    seen, xcd = set(), {}
    n = units * G
    if plan["xcd_group"] == 1:
        assert splits > 1 and units >= 8 and G > 1
        assert plan["workgroups"] == -(-units // 8) * 8 * G
    elif plan["xcd_group"] == 2:
        assert splits == 1 and n >= 16
        assert plan["workgroups"] == -(-n // 8) * 8
    else:
        assert plan["workgroups"] == n
    runs = {}
    for bid in range(plan["workgroups"]):
        if plan["xcd_group"] == 2:
            r = (bid & 7) * (plan["workgroups"] >> 3) + (bid >> 3)
            if r >= n:
                continue
            runs.setdefault(bid & 7, []).append(r)
            hh = r % (Hkv * HB)
            r //= Hkv * HB
            split, qt = r % splits, n_qblocks - 1 - r // splits
            h, hb = hh // HB, hh % HB
        elif plan["xcd_group"] == 1:
            lo, rest = bid & 7, bid >> 3
            g, unit = rest % G, (rest // G) * 8 + lo
            if unit >= units:
                continue
            h, split, hb, qt = unit % Hkv, unit // Hkv, g % HB, n_qblocks - 1 - g // HB
        else:
            r = bid
            hh = r % (Hkv * HB)
            r //= Hkv * HB
            split, qt = r % splits, n_qblocks - 1 - r // splits
            h, hb = hh // HB, hh % HB
        assert 0 <= qt < n_qblocks
        key = (h, hb, split, qt)
        assert key not in seen
        seen.add(key)
        xcd.setdefault((h, split), set()).add(bid % 8)
    assert len(seen) == units * G
    if plan["xcd_group"] == 1:
        assert all(len(v) == 1 for v in xcd.values())
    if plan["xcd_group"] == 2:
        for ids in runs.values():
            assert ids == list(range(ids[0], ids[0] + len(ids)))


def check_prefill(cfg, P, plan):
    """prefill_kernel: workgroup (qt, split) of a head block covers key tiles
    [t_begin + split*tps, min(t_end, t_begin + (split+1)*tps)) of its query
    block's range [t_begin, t_end)."""
    D, S, Hq, Hkv, W, causal = (cfg.head_dim, cfg.query_len, cfg.num_heads, cfg.kv_heads, cfg.window,
                                cfg.causal)
    assert plan["path"] == _ffi.KERNEL_PREFILL_BF16
    BN, WGQ = plan["tile_keys"], plan["workgroup_queries"]
    splits, tps = plan["splits"], plan["tiles_per_split"]
    assert TILE_ALIGN % BN == 0
    key_total = P + S
    n_qblocks = -(-S // WGQ)
    rb, kw = plan["heads_per_block"], plan["block_waves"]
    # four waves per workgroup of 32 queries each (16 at head_dim 256); wave
    # pairs (kw = 2) put two waves on each block
    assert kw in (1, 2) and rb * WGQ * kw == (64 if D >= 256 else 128)
    assert plan["head_blocks"] * rb == Hq // Hkv
    check_prefill_grid(plan, n_qblocks, Hkv, plan["head_blocks"], splits)
    P8 = P & ~(TILE_ALIGN - 1)
    cap_stage = ((P + S + TILE_ALIGN - 1) & ~(TILE_ALIGN - 1)) - P8
    assert plan["stage_bytes"] == 2 * Hkv * cap_stage * D * 2
    if splits > 1:
        assert plan["partial_bytes"] == splits * S * Hq * (D + 2) * 4
    else:
        assert plan["partial_bytes"] == 0
    widest = 0
    for qt in range(n_qblocks):
        p0 = qt * WGQ
        key_end = min(key_total, P + min(S, p0 + WGQ)) if causal else key_total
        key_begin = max(0, P + p0 - W + 1) if W > 0 else 0
        t_begin, t_end = key_begin // BN, -(-key_end // BN)
        widest = max(widest, t_end - t_begin)
        # the keys any query of the block may see lie inside [t_begin, t_end) tiles
        for i in (p0, min(S, p0 + WGQ) - 1):
            lo = max(0, P + i - W + 1) if W > 0 else 0
            hi = P + i if causal else key_total - 1
            if lo <= hi:
                assert t_begin * BN <= lo and hi < t_end * BN
        # the splits cover every tile of the block's range, once
        seen = []
        for split in range(splits):
            tb = t_begin + (split * tps if splits > 1 else 0)
            te = min(t_end, tb + tps) if splits > 1 else t_end
            seen.extend(range(tb, te))
        assert seen == list(range(t_begin, t_end)), (qt, t_begin, t_end, splits, tps)
        # wave pairs: in each split, wave kh of the pair takes tile kw*T + kh of
        # super-tiles T in [tb // kw, ceil(te / kw)), hidden outside [tb, te),
        # and copies min(kw*T + i, te - 1): every tile once, every copy inside
        for split in range(splits):
            tb = t_begin + (split * tps if splits > 1 else 0)
            te = min(t_end, tb + tps) if splits > 1 else t_end
            if tb >= te:
                continue
            taken = sorted(kw * T + kh for T in range(tb // kw, -(-te // kw)) for kh in range(kw)
                           if tb <= kw * T + kh < te)
            assert taken == list(range(tb, te))
            copied = {min(kw * T + i, te - 1) for T in range(tb // kw, -(-te // kw)) for i in range(kw)}
            assert min(copied) >= tb - (kw - 1) and max(copied) == te - 1
        # staged rows the block reads stay inside the staging buffer
        if t_end * BN > P8:
            assert t_end * BN - P8 <= cap_stage
    assert widest == plan["max_tiles"]


BASELINE_DECODE = [  # (name, Hq, Hkv, D, past lens, window)
    ("cfg0 llama-1B @512", 32, 8, 64, [512], 0),
    ("cfg1 llama-1B @2048..2175", 32, 8, 64, [2175], 0),
    ("cfg2b llama-3B @8192 b1", 24, 8, 128, [8192], 0),
    ("cfg2b llama-3B @8192 b16", 24, 8, 128, [8192] * 16, 0),
    ("cfg3 gemma-1B global @32768", 4, 1, 256, [32768], 0),
    ("cfg3 gemma-1B local W512", 4, 1, 256, [32768], 512),
    ("cfg4 gemma-4B global @16640", 8, 4, 256, [16640], 0),
    ("cfg4 gemma-4B local W1024", 8, 4, 256, [16640], 1024),
    ("ragged batch of 40", 24, 8, 128, [random.Random(3).randrange(0, 9000) for _ in range(40)], 0),
    ("one long, fifteen short", 32, 8, 256, [16384] + [64] * 15, 0),
    ("first token", 24, 8, 128, [0, 0, 0], 0),
]

BASELINE_PREFILL = [  # (name, S, P, Hq, Hkv, D, window, causal)
    ("cfg1 llama-1B prefill 2048", 2048, 0, 32, 8, 64, 0, True),
    ("cfg2a llama-3B prefill 4096", 4096, 0, 24, 8, 128, 0, True),
    ("cfg3 gemma-1B prefill global", 4096, 0, 4, 1, 256, 0, True),
    ("cfg3 gemma-1B prefill local W512", 4096, 0, 4, 1, 256, 512, True),
    ("cfg4 gemma-4B chunk global", 128, 16384, 8, 4, 256, 0, True),
    ("cfg4 gemma-4B chunk local W1024", 128, 16384, 8, 4, 256, 1024, True),
    # windowed non-causal chunks whose split plan once covered too few tiles
    ("non-causal W512 over 4100", 256, 4100, 32, 8, 64, 512, False),
    ("non-causal W1024 over 8000", 512, 8000, 32, 8, 128, 1024, False),
    ("non-causal W256 d256", 200, 3000, 8, 4, 256, 256, False),
    # wave pairs (head_dim-64 causal prompts): R = 4, 2, 3 and 1, ragged lengths
    ("pairs llama-1B prompt 1024", 1024, 0, 32, 8, 64, 0, True),
    ("pairs R=2 prompt 333", 333, 0, 16, 8, 64, 0, True),
    ("pairs R=3 prompt 700", 700, 0, 24, 8, 64, 0, True),
    ("pairs R=1 prompt 129 after 7", 129, 7, 8, 8, 64, 0, True),
    ("llama-1B chunk 128 on 2048", 128, 2048, 32, 8, 64, 0, True),
    ("llama-3B chunk 256 on 8192", 256, 8192, 24, 8, 128, 0, True),
    ("llama-3B chunk 64 on 8192", 64, 8192, 24, 8, 128, 0, True),
    ("llama-3B tp8 share prompt 4096", 4096, 0, 3, 1, 128, 0, True),
    ("pairs with key splits, 4/1 heads 2048", 2048, 0, 4, 1, 64, 0, True),
]


@pytest.mark.parametrize("name,Hq,Hkv,D,past,W", BASELINE_DECODE, ids=[c[0] for c in BASELINE_DECODE])
@pytest.mark.parametrize("noalloc", [False, True])
def test_decode_plan_covers_every_key(name, Hq, Hkv, D, past, W, noalloc):
    cfg = KvAttentionConfig(1, Hq, Hkv, D, True, W)
    plan = plan_attention(cfg, past, noalloc=noalloc)
    for b0 in range(0, len(past), MAX_DECODE_BATCH):  # each launch of <= 16 sequences
        chunk = past[b0:b0 + MAX_DECODE_BATCH]
        check_decode(cfg, chunk, plan_attention(cfg, chunk, noalloc=noalloc), noalloc)
    assert plan["partial_bytes"] >= max(
        plan_attention(cfg, past[b0:b0 + MAX_DECODE_BATCH], noalloc=noalloc)["partial_bytes"]
        for b0 in range(0, len(past), MAX_DECODE_BATCH))


def test_decode_token_split_only_when_two_entries_fit():
    cfg = KvAttentionConfig(1, 24, 8, 128, True, 0)
    assert plan_attention(cfg, [8192])["token_split"] == 1
    assert plan_attention(cfg, [8192], noalloc=True)["token_split"] == 1
    # batch 16: the grid already fills a round of workgroup slots
    assert plan_attention(cfg, [8192] * 16)["token_split"] == 0
    # 15 sequences x 512 heads x (256 + 2) floats fill the scratch array once: the token goes to split 0
    wide = KvAttentionConfig(1, 512, 512, 256, True, 0)
    plan = plan_attention(wide, [4] * 15, noalloc=True)
    assert plan["token_split"] == 0 and plan["splits"] == 1


def test_noalloc_plan_coarsens_splits_to_the_scratch_array():
    cfg = KvAttentionConfig(1, 32, 8, 256, True, 0)
    past = [16384] + [64] * 15
    wide = plan_attention(cfg, past)
    narrow = plan_attention(cfg, past, noalloc=True)
    assert wide["partial_bytes"] > SCRATCH_BYTES >= narrow["partial_bytes"]
    assert narrow["splits"] < wide["splits"]
    check_decode(cfg, past, narrow, noalloc=True)


def test_noalloc_plan_rejects_partials_beyond_the_scratch_array():
    # 16 sequences x 512 heads x (256 + 2) floats = 8.45 MB > 8 MiB even unsplit
    cfg = KvAttentionConfig(1, 512, 512, 256, True, 0)
    with pytest.raises(ShapeError):
        plan_attention(cfg, [4] * 16, noalloc=True)
    plan_attention(cfg, [4] * 15, noalloc=True)  # 7.9 MB fits


@pytest.mark.parametrize("name,S,P,Hq,Hkv,D,W,causal", BASELINE_PREFILL, ids=[c[0] for c in BASELINE_PREFILL])
def test_prefill_plan_covers_every_key(name, S, P, Hq, Hkv, D, W, causal):
    cfg = KvAttentionConfig(S, Hq, Hkv, D, causal, W)
    check_prefill(cfg, P, plan_attention(cfg, [P]))


def test_split_prefill_groups_shared_keys_on_one_xcd():
    # Gemma-3-4B chunk: 4 KV heads x 31 splits, two 64-query workgroups per split
    plan = plan_attention(KvAttentionConfig(128, 8, 4, 256, True, 0), [16384])
    assert plan["splits"] > 1 and plan["xcd_group"] == 1
    # Llama-3.2-3B chunk: three head blocks of one KV head read the same keys
    plan = plan_attention(KvAttentionConfig(128, 24, 8, 128, True, 0), [8192])
    assert plan["splits"] > 1 and plan["xcd_group"] == 1
    # unsplit prefill keeps the longest-first order
    assert plan_attention(KvAttentionConfig(4096, 24, 8, 128, True, 0), [0])["xcd_group"] == 0
    # Gemma-3-1B local W512 (one KV head, unsplit): adjacent query blocks per XCD
    plan = plan_attention(KvAttentionConfig(4096, 4, 1, 256, True, 512), [0])
    assert plan["splits"] == 1 and plan["xcd_group"] == 2


def test_prefill_plan_sweep():
    rng = random.Random(20261202)
    for _ in range(300):
        D = rng.choice([64, 128, 256])
        Hkv = rng.choice([1, 2, 4, 8])
        Hq = Hkv * rng.choice([1, 2, 3, 4, 8])
        S = rng.choice([2, 33, 64, 128, 257, 1000, 4096])
        P = rng.choice([0, 5, 64, 100, 2048, 4100, 16384])
        W = rng.choice([0, 0, 1, 17, 64, 512, 1024, 5000])
        causal = rng.random() < 0.7
        cus = rng.choice([256, 80, 304])
        cfg = KvAttentionConfig(S, Hq, Hkv, D, causal, W)
        check_prefill(cfg, P, plan_attention(cfg, [P], compute_units=cus))


def test_decode_plan_sweep():
    rng = random.Random(7)
    for _ in range(200):
        D = rng.choice([64, 128, 256])
        Hkv = rng.choice([1, 2, 4, 8])
        Hq = Hkv * rng.choice([1, 2, 3, 4, 5, 8])
        B = rng.choice([1, 2, 7, 16])
        past = [rng.choice([0, 1, 47, 512, 8191, 32768]) for _ in range(B)]
        W = rng.choice([0, 0, 1, 100, 1024])
        cfg = KvAttentionConfig(1, Hq, Hkv, D, True, W)
        for noalloc in (False, True):
            check_decode(cfg, past, plan_attention(cfg, past, noalloc=noalloc), noalloc)


def test_plan_paths():
    assert plan_attention(KvAttentionConfig(1, 6, 3, 48, True), [10])["path"] == _ffi.KERNEL_GENERIC
    assert plan_attention(KvAttentionConfig(8, 6, 3, 128, True), [10],
                          precision=_ffi.PREFILL_F32)["path"] == _ffi.KERNEL_GENERIC
    assert plan_attention(KvAttentionConfig(8, 6, 3, 128, True), [10])["path"] == _ffi.KERNEL_PREFILL_BF16


def test_causal_prompt_plans_pair_waves_and_skip_key_splits():
    """Head_dim-64 causal prompts pair waves while the paired grid fits one
    round of workgroup slots; causal prompts at head_dim 64/128 never take key
    splits; chunks over longer caches keep single waves and key splits."""
    p = plan_attention(KvAttentionConfig(1024, 32, 8, 64, True, 0), [0])
    assert (p["block_waves"], p["splits"], p["workgroups"]) == (2, 1, 512)
    assert (p["heads_per_block"], p["workgroup_queries"]) == (2, 32)
    p = plan_attention(KvAttentionConfig(2048, 32, 8, 64, True, 0), [0])
    assert (p["block_waves"], p["splits"], p["workgroups"]) == (1, 1, 512)
    p = plan_attention(KvAttentionConfig(700, 24, 8, 64, True, 0), [0])
    assert (p["block_waves"], p["heads_per_block"], p["workgroup_queries"]) == (2, 1, 64)
    p = plan_attention(KvAttentionConfig(1024, 24, 8, 128, True, 0), [0])
    assert (p["block_waves"], p["splits"]) == (1, 1)
    p = plan_attention(KvAttentionConfig(512, 24, 8, 128, True, 0), [0])  # 96 workgroups of 8 tiles
    assert (p["block_waves"], p["splits"]) == (1, 1)
    # one GPU's share of a head split (3 query heads, 1 KV head): 32
    # workgroups unsplit, so key splits still fill the GPU
    p = plan_attention(KvAttentionConfig(4096, 3, 1, 128, True, 0), [0])
    assert p["block_waves"] == 1 and p["splits"] > 1
    p = plan_attention(KvAttentionConfig(2048, 4, 1, 64, True, 0), [0])  # 128 paired workgroups
    assert p["block_waves"] == 2 and p["splits"] > 1
    p = plan_attention(KvAttentionConfig(100, 32, 8, 64, True, 0), [0])  # fewer than two tiles
    assert p["block_waves"] == 1
    p = plan_attention(KvAttentionConfig(128, 32, 8, 64, True, 0), [2048])
    assert p["block_waves"] == 1 and p["splits"] > 1
    # head_dim-256 causal prompts: one and a half rounds (Gemma-3-1B global)
    p = plan_attention(KvAttentionConfig(4096, 4, 1, 256, True, 0), [0])
    assert (p["splits"], p["workgroups"]) == (3, 768)
    # head_dim-64/128 chunks aim at three quarters of a round of slots
    for S, P, want in ((256, 8192, 8), (512, 4096, 4), (64, 8192, 16)):
        p = plan_attention(KvAttentionConfig(S, 24, 8, 128, True, 0), [P])
        # (the split count is the tile range over whole tiles per split)
        assert want - 1 <= p["splits"] <= want and p["workgroups"] <= 384, (S, P, p["splits"])
    p = plan_attention(KvAttentionConfig(1024, 32, 8, 64, False, 0), [0])
    assert p["block_waves"] == 1
