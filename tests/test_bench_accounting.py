"""The bench's algorithmic accounting against the work figures of the
BASELINE configs (bytes of the visible K/V per decode layer, unmasked
(query, key) pairs and FLOP per prefill layer), so that the GB/s and TFLOP/s
it reports are credited on the stated units. Runs without a GPU."""
import bench


def test_decode_bytes_per_layer():
    # Llama-3.2-3B at 8192 cached keys: 8193 x 8 x 128 x 4 x 2 + q/out + append
    assert bench.decode_bytes(8193) == 67_149_824
    # Llama-3.2-1B at 512 cached keys: 2 x 513 x 8 x 64 x 4 = 2.10 MB, plus 20 KB
    assert bench.decode_bytes(513, 32, 8, 64) == 2 * 513 * 8 * 64 * 4 + 32 * 64 * 8 + 2 * 8 * 64 * 4
    # Gemma-3-1B global at 32768 (1 KV head, d 256): 67.1 MB of K/V
    assert abs(bench.decode_bytes(32769, 4, 1, 256) - 67.1e6) < 0.1e6
    # Gemma-3-4B global at 16513 keys: 135.3 MB of f32 K/V
    assert abs(bench.decode_bytes(16513, 8, 4, 256) - 135.3e6) < 0.1e6


def test_prefill_pairs_and_flop():
    # causal, no cache: S(S+1)/2
    assert bench.visible_pairs(4096, 0, 0) == 4096 * 4097 // 2
    assert bench.prefill_flops(4096) == 103_104_380_928
    assert round(bench.prefill_flops(2048, 32, 64) / 1e9, 2) == 17.19
    # Gemma-3-1B local layers, window 512: sum of min(i + 1, 512)
    assert bench.visible_pairs(4096, 0, 512) == 1_966_336
    assert round(4.0 * 256 * 4 * 1_966_336 / 1e9, 2) == 8.05
    # a 128-token chunk after 16384 cached keys: S*P + S(S+1)/2
    assert bench.visible_pairs(128, 16384, 0) == 128 * 16384 + 8256
    assert round(4.0 * 256 * 8 * bench.visible_pairs(128, 16384, 0) / 1e9, 2) == 17.25
    # the same chunk in a W1024 layer: every query sees exactly the window
    assert bench.visible_pairs(128, 16384, 1024) == 128 * 1024


def test_config_cases_cover_every_other_baseline_config():
    # config 2 is the main bench; its cases here are one GPU's share of an 8-way head split
    assert {c[1] for c in bench.CONFIG_CASES if "tp8_share" not in c[0]} == {0, 1, 3, 4}
    shares = [c for c in bench.CONFIG_CASES if "tp8_share" in c[0]]
    assert shares and all(c[1] == 2 and (c[3], c[4], c[5]) == (24 // 8, 8 // 8, 128) for c in shares)


def test_traffic_profile_matches_the_planned_decode_launch():
    # roofline.traffic comes from profiles/decode_b1_hbm_traffic.md: its counts
    # must belong to the launch the library plans now (host arithmetic only)
    plan = bench.decode_plan()
    got = bench.measured_traffic(plan)
    assert got["profile_plan"] == plan, (got["profile_plan"], plan)
    assert got["stale"] is False and got["bytes"] is not None
    # within a few percent of the algorithmic bytes of one launch
    assert 1.0 <= got["bytes"] / bench.decode_bytes(8193) < 1.1


def test_stale_traffic_profile_is_withheld():
    plan = dict(bench.decode_plan())
    plan["splits"] += 1
    got = bench.measured_traffic(plan)
    assert got["stale"] is True and got["bytes"] is None
