"""The tune CLI's record keeping, without a GPU: the fastest successful candidate is kept per
context, failed candidates are left out of both records, contexts already in the files are
merged, and the files are rewritten whole after each context."""
import json

from mlc_decode_amd.tune import ALL_FILE, BEST_FILE, Measurement, TuneRecords, parse_args


def _m(ns, windows, error=None):
    return Measurement({"num_split": ns, "spread": True, "block_N": 64}, list(windows), error)


def test_records_keep_fastest_and_drop_failures(tmp_path):
    (tmp_path / BEST_FILE).write_text(json.dumps({"64": {"num_split": 1, "latency_us": 9.0}}))
    rec = TuneRecords(str(tmp_path))
    results = [_m(None, [12.0, 11.0, 30.0]), _m(2, [10.5, 10.7, 10.6]), _m(4, [], "RuntimeError: rejected"),
               _m(8, [10.9, 10.2, 10.4])]
    best = rec.update(4096, results)
    assert best == {"num_split": 8, "spread": True, "block_N": 64, "latency_us": 10.4}
    rec.save()
    saved_best = json.loads((tmp_path / BEST_FILE).read_text())
    saved_all = json.loads((tmp_path / ALL_FILE).read_text())
    assert sorted(saved_best) == ["4096", "64"]          # merged with the existing context
    assert [r["num_split"] for r in saved_all["4096"]] == [None, 2, 8]  # the failure is left out
    assert saved_all["4096"][0]["latency_us"] == 12.0    # median window, not the mean
    assert not list(tmp_path.glob("*.partial"))


def test_context_with_no_successful_candidate_is_skipped(tmp_path):
    rec = TuneRecords(str(tmp_path))
    assert rec.update(2048, [_m(1, [], "ValueError: bad")]) is None
    rec.save()
    assert json.loads((tmp_path / BEST_FILE).read_text()) == {}
    assert "FAILED" in _m(1, [], "ValueError: bad").describe()


def test_reference_flags_are_accepted():
    a = parse_args(["--kv-ctx", "2048", "4096", "--batch", "2", "--heads", "128", "--kv-heads", "1",
                    "--dim", "512", "--pe-dim", "64", "--warmup", "5", "--rep", "7"])
    assert a.kv_ctx == [2048, 4096] and a.batch == 2 and a.heads == 128 and a.rep == 7 and a.windows == 3
