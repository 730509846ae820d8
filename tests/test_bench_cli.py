"""bench.py's command-line contract that needs no GPU."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_refuses_more_than_one_gpu():
    # this build measures one GPU: --gpus N > 1 exits with status 2 and says so
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], cwd=ROOT,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2, r.stderr
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_bench_refuses_a_split_count_outside_the_abi_range():
    # --decode-splits pins the Qwen3-32B split count; outside [1, 4096] it exits
    # with status 2 before touching a GPU
    for bad in ("0", "4097"):
        r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--decode-splits", bad],
                           cwd=ROOT, capture_output=True, text=True, timeout=120)
        assert r.returncode == 2, r.stderr
        assert "[1, 4096]" in r.stderr
        assert r.stdout == ""


def test_guarded_section_records_its_error():
    # a secondary section that raises leaves an error entry, not a missing line
    sys.path.insert(0, ROOT)
    import bench

    assert bench.guarded(lambda: {"us": 1.0}) == {"us": 1.0}
    r = bench.guarded(lambda: 1 / 0)
    assert r == {"error": "ZeroDivisionError: division by zero"}


def _fake_results():
    """Results shaped as bench.py's sections return them (numbers of a real
    run, rounded), every section present."""
    dist = {"p10_us": 21.4, "median_us": 21.45, "p90_us": 21.5, "calls_per_replay": 100,
            "replays": 20}

    def dec(ctx, step_us, split_us):
        return {"step_ms": step_us * 1e-3, "split_ms": split_us * 1e-3, "step_dist": dist,
                "split_dist": dist, "alg_bytes": 2 * 8 * ctx * 128 * 2 + 32768,
                "num_splits": 32, "default_splits": 32,
                "sweep_us": {8: 51.6, 16: 30.6, 32: step_us, 64: 24.7}}

    def pre(S, us):
        return {"ms": us * 1e-3, "flop": 4.0 * 32 * 128 * S * (S + 1) / 2, "dist": dist,
                "plan": {"form": 1, "name": "per-team, 128-row q blocks", "paired": True,
                         "workgroups": 256},
                "library": {"name": "torch sdpa", "ms": 3.3 * us * 1e-3, "max_abs_diff": 0.002}}

    sweep = {8192: dec(8192, 9.7, 7.5), 16384: dec(16384, 14.4, 12.2),
             32768: dec(32768, 23.5, 21.4)}
    psweep = {512: pre(512, 10.1), 2048: pre(2048, 40.2), 8192: pre(8192, 487.0)}
    eng_q = {"prefill_ms": 9.8, "decode_ms": 1.41, "tok_s": 709.8, "bytes_per_token": 2.59e9,
             "weight_bytes": 2490931712, "distinct_tokens": 256, "mean_ctx": 640.0}
    return {
        "decode32b_sweep": sweep, "decode32b": sweep[32768],
        "prefill_sweep": psweep, "prefill": psweep[2048],
        "decode4b": {"step_ms": 7.6e-3, "split_ms": 5.5e-3, "alg_bytes": 16793600,
                     "num_splits": 32, "graph_ms": 0.30},
        "shard": {"kv_head": {"step_ms": 0.0103, "split_ms": 0.0064, "alg_bytes": 16781312,
                              "num_splits": 128, "sweep_us": {32: 16.5, 128: 10.4}},
                  "merge_ms": 0.0022},
        "norm": {"ms": 0.0083, "alg_bytes": 50331648},
        "engine4b": {"prefill_ms": 7.4, "decode_ms": 1.75, "tok_s": 570.3,
                     "bytes_per_token": 8.14e9, "distinct_tokens": 253, "mean_ctx": 640.0,
                     "prefill_sweep_ms": {18: 3.2, 128: 5.5, 512: 7.1, 2048: 18.7, 8192: 75.3},
                     "attn_graph_ms": 0.24},
        "engine32b": {"weight_bytes": 63.99e9,
                      "requests": [{"pp": 18, "tg": 128, "prefill_ms": 19.7, "e2e_ms": 1326.7,
                                    "decode_ms_per_token": 10.29, "request_gen_tps": 96.5,
                                    "reference_b200_request_gen_tps": 79.9}]},
        "engine4b_q4km": eng_q, "engine4b_q5km": dict(eng_q, tok_s=652.6),
    }


def test_line_assembly_from_every_section():
    """The JSON line's contract, built from results of every section (the
    assembly runs after minutes of GPU work, so a key error there would cost
    the whole line): the contract fields, the roofline and cpu_baseline
    objects, and one entry per section."""
    import json

    sys.path.insert(0, ROOT)
    import bench

    cpu = {"value": 2.19, "unit": "GB/s", "cores": 16, "kind": "port", "sample": "s",
           "single_thread": {"value": 0.14, "unit": "GB/s", "cores": 1}}
    line = bench.assemble_line(_fake_results(), 20, 5, cpu)
    json.loads(json.dumps(line))
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
              "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config"):
        assert k in line, k
    assert line["n_gpus"] == 1 and line["vs_baseline"] is None and line["unit"] == "GB/s"
    assert abs(line["value"] - 134250496 / 23.5e-6 / 1e9) < 0.1
    assert set(line["roofline"]) >= {"bound", "achieved", "peak", "unit", "frac", "traffic"}
    assert set(line["cpu_baseline"]) >= {"value", "unit", "cores", "kind", "sample"}
    for k in ("decode32b_sweep", "prefill", "prefill_sweep", "decode4b", "shard",
              "qk_norm_rope_kv", "engine4b", "engine32b", "engine4b_q4km", "engine4b_q5km"):
        assert k in line and "error" not in line[k], k
    assert set(line["engine4b"]["prefill_sweep"]) == {"18", "128", "512", "2048", "8192"}


def test_line_assembly_with_failed_sections():
    """Failed secondary sections carry their error in the line; the headline
    fields stay."""
    sys.path.insert(0, ROOT)
    import bench

    res = _fake_results()
    for k in ("engine4b", "engine32b", "norm", "shard"):
        res[k] = {"error": "RuntimeError: x"}
    del res["prefill"], res["prefill_sweep"]
    res["prefill_error"] = {"error": "RuntimeError: y"}
    line = bench.assemble_line(res, 20, 5, None)
    assert line["engine4b"] == {"error": "RuntimeError: x"}
    assert line["qk_norm_rope_kv"] == {"error": "RuntimeError: x"}
    assert line["prefill"] == {"error": "RuntimeError: y"}
    assert "value" in line and "roofline" in line and "cpu_baseline" not in line
