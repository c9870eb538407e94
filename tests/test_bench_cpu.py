"""bench.py and the entry points on the CPU: the contract pieces that need no GPU."""
import importlib
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    return importlib.import_module("bench")


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr or "single" in r.stderr
    assert r.stdout == ""


def test_algorithmic_work_matches_the_workload_definitions():
    b = _bench()
    # decode GEMV [1,3840] x [15360,3840]: nibbles + bf16 scale/bias per 64 + x + y
    assert b.q4_bytes(15360, 3840) == 29_491_200 + 3_686_400
    assert b.gemv_bytes(1, 15360, 3840) == 33_216_000
    # quantize/pack [15360,3840]: bf16 read + Q4 written
    assert 2 * 15360 * 3840 + b.q4_bytes(15360, 3840) == 151_142_400
    # prefill: 2 M sum(n k) over the seven projections of a layer
    from hyperion_amd import synthetic as syn
    nk = sum(n * k for n, k in syn.LAYER_SHAPES.values())
    assert nk == 224_133_120                     # weights per layer
    assert 2 * 2048 * nk == 918_049_259_520      # 9.180e11 flop at M = 2048
    assert 2 * 512 * nk == 229_512_314_880       # 2.295e11 flop at M = 512


def test_roofline_traffic_comes_from_the_committed_counter_summary():
    """roofline.traffic is the committed record's scaled FETCH_SIZE + WRITE_SIZE, which lies
    within 5% above the algorithmic bytes (every weight byte read once)."""
    import json
    import re
    b = _bench()
    text = open(os.path.join(ROOT, "profiles", "decode_gemv_traffic.md")).read()
    rec = json.loads(re.search(r"```json\s*(\{.*?\})\s*```", text, flags=re.S).group(1))
    assert b.measured_traffic() == rec["hbm_bytes_per_launch"]
    assert rec["hbm_bytes_per_launch"] == rec["hbm_read_bytes_per_launch"] + rec["hbm_write_bytes_per_launch"]
    assert rec["algorithmic_bytes_per_launch"] == b.gemv_bytes(1, 15360, 3840)
    assert 1.0 <= rec["hbm_bytes_per_launch"] / rec["algorithmic_bytes_per_launch"] <= 1.05


def test_entry_points_exist():
    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    g = importlib.import_module("__graft_entry__")
    assert callable(g.build) and callable(g.smoke)


def test_cold_rotation_never_rereads_a_copy_within_the_mall():
    """Simulate the bench's index arithmetic: every timed launch on copy c must be
    separated from the previous read of c (warm-up included) by more than 256 MiB of
    other weight bytes, for any steps/warmup at the default copy counts."""
    b = _bench()
    per_copy = b.q4_bytes(15360, 3840)
    calls = []

    class _Stream:
        def synchronize(self):
            pass

    class _Event:
        def record(self, _s):
            pass

        def elapsed_ms(self, _e):
            return 1.0

        def close(self):
            pass

    saved = b.hy.Event
    b.hy.Event = _Event
    try:
        for steps, warmup in ((20, 5), (200, 20), (7, 0), (1, 30)):
            calls.clear()
            b.time_launches(_Stream(), lambda i: calls.append(i), steps, warmup)
            copies = 24
            assert b.cold_rotation_ok(copies, per_copy)
            last = {}
            for pos, i in enumerate(calls):
                c = i % copies
                if pos >= warmup and c in last:
                    between = (pos - last[c] - 1) * per_copy
                    assert between > b.MALL_BYTES, (steps, warmup, pos)
                last[c] = pos
    finally:
        b.hy.Event = saved
    assert not b.cold_rotation_ok(8, per_copy)   # 7 x 33 MB < 256 MiB: refused
