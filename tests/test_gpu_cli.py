"""The check CLI (``python -m mlc_decode_amd.check``, the reference's ``scripts/check_mla.py``
columns) runs end to end and reports errors within the parity bar."""
import pytest

pytestmark = pytest.mark.gpu


def test_check_cli_rows(gpu, capsys):
    from mlc_decode_amd import check
    rows = check.main(["--kv-ctx", "33", "4095", "--warmup", "1", "--rep", "3"])
    out = capsys.readouterr().out
    assert "max_abs_err" in out and "cos_sim" in out
    assert [ctx for ctx, _ in rows] == [33, 4095]
    for ctx, r in rows:
        assert r["max_abs_err"] <= 1e-2 and r["cos_sim"] >= 0.99999, (ctx, r)
        assert r["our_us"] > 0 and r["torch_us"] > 0


def test_tune_cli_records(gpu, tmp_path, capsys):
    """``python -m mlc_decode_amd.tune`` (scripts/tune_best.py's flags and outputs): every
    candidate of mla_autotune_configs is timed and kept in mla_tune_all.json, and
    mla_best_configs.json holds the fastest one per context; a second run merges."""
    import json

    from mlc_decode_amd import tune
    from mla_decode import mla_autotune_configs
    assert tune.main(["--kv-ctx", "130", "--warmup", "1", "--rep", "3", "--out-dir", str(tmp_path)]) == 0
    assert tune.main(["--kv-ctx", "700", "--warmup", "1", "--rep", "3", "--out-dir", str(tmp_path)]) == 0
    best = json.loads((tmp_path / "mla_best_configs.json").read_text())
    rows = json.loads((tmp_path / "mla_tune_all.json").read_text())
    assert sorted(best) == sorted(rows) == ["130", "700"]
    for ctx in (130, 700):
        cands = mla_autotune_configs(1, 16, 1, ctx, 512, 64)
        got = rows[str(ctx)]
        assert [r["num_split"] for r in got] == [c["num_split"] for c in cands]
        assert all(r["latency_us"] > 0 for r in got)
        assert best[str(ctx)]["latency_us"] == min(r["latency_us"] for r in got)
    assert "wrote" in capsys.readouterr().out
