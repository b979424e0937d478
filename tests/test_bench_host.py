"""Host-side logic of bench.py (no GPU): the counter-summary staleness key
and the traffic lookup."""
import importlib.util
import json
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_code_hash_ignores_comments_only():
    b = _bench()
    src = "int f(int x) {\n  // twice\n  return 2 * x;  /* doubled */\n}\n"
    same = "int f(int x) {\n  // multiply by two\n\n  return 2 * x;\n}\n"
    other = "int f(int x) {\n  // twice\n  return 3 * x;\n}\n"
    assert b._source_sha(src) == b._source_sha(same)
    assert b._source_sha(src) != b._source_sha(other)


def test_traffic_reported_only_for_the_measured_code(tmp_path, monkeypatch):
    b = _bench()
    with open(os.path.join(ROOT, "profiles", "traffic_cfg2.json")) as f:
        rec = json.load(f)
    prof = tmp_path / "profiles"
    prof.mkdir()
    monkeypatch.setattr(b, "ROOT", str(tmp_path))
    rec["decode_source_sha256"] = b._source_sha()
    (prof / "traffic_cfg2.json").write_text(json.dumps(rec))
    assert b._traffic("cfg2") == rec["hbm_bytes_per_launch"]
    rec["decode_source_sha256"] = "0" * 16
    (prof / "traffic_cfg2.json").write_text(json.dumps(rec))
    assert b._traffic("cfg2") is None
