"""The benchmark's stdout contract without a GPU: one JSON line, short enough
for a driver that keeps a few KB of stdout, carrying the headline fields, the
dominant kernel's roofline and the CPU baseline; the per-launch tables go to
stderr and to --detail."""
import json
import types

import bench


def fake_update(workload, kernel, launches=40):
    rows = [{"name": f"kernel_{i}", "layout": [1, 0], "shape": [32768, 256, 400], "ms": 0.07, "ms_alone": 0.069,
             "count": 32, "bound": "mfma", "achieved": 90.1, "frac": 0.57} for i in range(launches)]
    return {
        "value": 24512345.678, "unit": "samples/s", "n_gpus": 1, "steps": 20, "warmup": 2,
        "ms_per_step": 10.694321, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic seeded rollout, random-init network",
        "config": {"workload": workload, "T": 128, "N": 2048, "obs": 400, "epochs": 4, "minibatches": 8,
                   "minibatch": 32768, "global_batch": 262144, "graph": True},
        "roofline": {"bound": "mfma", "achieved": 90.43, "peak": 157.3, "unit": "TFLOP/s", "frac": 0.5749,
                     "traffic": 117934080.0, "kernel": kernel, "avg_ms": 0.0742, "avg_ms_alone": 0.0731,
                     "share_of_update": 0.2213},
        "launches": rows, "launch_sum_ms": 10.5,
        "cpu_baseline": {"value": 101234.5, "unit": "samples/s", "cores": 16, "kind": "port",
                         "sample": "oracle restatement in float32 numpy: bootstrap forward, GAE over the full "
                                   "[128,2048] rollout and the 4 epoch permutations (1.23 s), plus 9 of the 32 "
                                   "minibatch steps of 32768 rows (gather, forward, backward, clip, Adam; 11.2 s), "
                                   "extrapolated to one update"},
    }


def test_headline_line_is_short_and_complete(capsys, tmp_path):
    out = {"metric": "PPO learner samples/sec on 1 MI355X + % of HBM/MFMA roofline per kernel",
           **fake_update("config 2: discrete-anakin", "ppo_gemm_f32 layout=[1, 0] MNK=[400, 256, 32768]")}
    full = [fake_update(f"config {c}: workload-name-{c}",
                        "ppo_gemm_bf16s_dw_group layout=[1, 0] MNK=[8268, 512, 8192, 4]") for c in (3, 4, 5, 6)]
    out["configs"] = [bench.compact_config(m) for m in full]
    out["_configs_full"] = full
    detail = tmp_path / "detail.json"
    bench.emit(out, types.SimpleNamespace(detail=str(detail)))
    captured = capsys.readouterr()
    lines = [ln for ln in captured.out.splitlines() if ln.strip()]
    assert len(lines) == 1
    assert len(lines[0].encode()) < 2000, len(lines[0].encode())
    line = json.loads(lines[0])
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
              "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline", "configs"):
        assert k in line, k
    assert "launches" not in line
    for k in ("bound", "achieved", "peak", "unit", "frac", "traffic", "kernel"):
        assert k in line["roofline"], k
    for k in ("value", "unit", "cores", "kind", "sample"):
        assert k in line["cpu_baseline"], k
    assert len(line["configs"]) == 4
    for c in line["configs"]:
        assert set(c) >= {"workload", "value", "ms_per_step", "frac", "kernel", "cpu"}
    # the launch tables are kept in the detail file and on stderr
    d = json.loads(detail.read_text())
    assert len(d["headline"]["launches"]) == 40 and len(d["configs"]) == 4
    assert "[bench] detail " in captured.err
