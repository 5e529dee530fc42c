"""CPU test of bench.py's result line: it carries the contract's fields and
stays short enough for a log tail to keep whole, however many components
the run measured."""
import importlib.util
import json
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    m = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(m)
    return m


def _components(n):
    names = list(_bench().NORTH_STAR_COMPONENTS) + [f"component_with_a_long_name_{i}" for i in range(n)]
    out = []
    for i, nm in enumerate(names):
        out.append({"name": nm, "ms": 0.0123 + i, "value": 1234.5678, "unit": "GB/s", "frac": 0.5678,
                    "bound": "hbm",
                    "cpu_baseline": {"value": 1.0, "unit": "GB/s", "cores": 8, "kind": "port",
                                     "sample": "x" * 400}})
    return out


def test_line_fields_and_size():
    b = _bench()
    h = {"value": 147.04, "ms_per_step": 0.935, "achieved": 147.3}
    cpu = {"value": 0.0123, "unit": "TFLOP/s", "cores": 1, "kind": "port", "sample": "s" * 1500}
    host = {"nproc": 128, "cpu_model": "AMD EPYC " + "y" * 60, "ram_gib": 1511.9, "rocm": "7.2.0",
            "torch": "2.10.0", "gpu": "AMD Instinct MI355X (gfx950, 256 CUs, 288 GiB)",
            "clocks_after_run": "z" * 1200}
    line = b.headline_line(20, 5, h, cpu, 470000000, host, _components(60), "gpurun_out/bench_detail.json")
    text = json.dumps(line)
    assert len(text) <= b.LINE_LIMIT, len(text)
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
              "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert k in line
    for k in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert k in line["roofline"]
    for k in ("value", "unit", "cores", "kind", "sample"):
        assert k in line["cpu_baseline"]
    assert line["roofline"]["frac"] == round(147.3 / 157.3, 4)
    # every north-star component is summarized, nothing else is
    assert sorted(line["north_star"]) == sorted(b.NORTH_STAR_COMPONENTS)
    assert line["components"]["count"] == len(b.NORTH_STAR_COMPONENTS) + 60
    assert "clocks_after_run" not in line["host"]


def test_line_without_cpu_or_components():
    b = _bench()
    h = {"value": 1.0, "ms_per_step": 1.0, "achieved": 1.0}
    line = b.headline_line(5, 1, h, None, None, {}, [], "d.json")
    assert line["cpu_baseline"] is None and line["north_star"] == {}
    assert len(json.dumps(line)) <= b.LINE_LIMIT
