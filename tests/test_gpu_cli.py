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
