"""Tuning-table (schema 1) and policy (schema 3) formats, no GPU."""
import json
from pathlib import Path

import pytest

from lich_amd import hierarchical_policy as HP
from lich_amd import tuning as TU
from lich_amd.kernels import KernelConfig

EXCERPT = Path(__file__).parent / "golden" / "policy_profile_excerpt.json"


def test_table_round_trip_and_lookup(tmp_path):
    e1 = TU.TuningEntry(TU.TuningKey("prediction", 64, 784, 128, "tanh", "float16"), KernelConfig(tile=3), 0.0123, False)
    e2 = TU.TuningEntry(TU.TuningKey("weight", 64, 64, 128, "tanh", "float16"),
                        KernelConfig(block_m=64, block_n=128, block_k=16, threads=128, num_stages=2), None, None)
    t = TU.TuningTable.from_entries([e1, e2])
    p = tmp_path / "t.json"
    t.to_json(p, device="MI355X", capability=(9, 5))
    payload = json.loads(p.read_text())
    assert payload["schema_version"] == 1 and payload["capability"] == [9, 5]
    # a config without a tile id serialises with the reference's fields only
    assert "tile" not in payload["entries"][1]["config"] and payload["entries"][0]["config"]["tile"] == 3
    back = TU.TuningTable.from_json(p)
    assert back == t
    assert back.lookup(kind="prediction", M=64, K=784, B=128, activation="tanh", dtype="float16").tile == 3
    assert back.lookup(kind="prediction", M=64, K=784, B=64, activation="tanh", dtype="float16") is None
    payload["schema_version"] = 2
    p.write_text(json.dumps(payload))
    with pytest.raises(ValueError, match="Unsupported tuning schema"):
        TU.TuningTable.from_json(p)


def test_unknown_config_fields_are_ignored():
    cfg = TU.config_from_dict({"block_m": 64, "block_n": 64, "warp_layout": "8x1"})
    assert cfg.block_m == 64 and cfg.tile_id() == 1


def test_kernel_signature_reproduces_the_reference_fingerprint():
    """The reference recorded kernel_signature for this profile's rows; the
    same rows must give the same fingerprint, or its execution entries would
    never resolve."""
    ex = json.loads(EXCERPT.read_text())
    prof = ex["kernel_profiles"][0]
    assert HP.kernel_signature(prof["kernel_entries"]) == prof["kernel_signature"]
    # row order does not matter, a changed config does
    rows = list(reversed(prof["kernel_entries"]))
    assert HP.kernel_signature(rows) == prof["kernel_signature"]
    rows[0] = dict(rows[0], config=dict(rows[0]["config"], threads=rows[0]["config"]["threads"] * 2))
    assert HP.kernel_signature(rows) != prof["kernel_signature"]


def test_policy_lookups_follow_the_reference_precedence():
    ex = json.loads(EXCERPT.read_text())
    pol = HP.HierarchicalPolicy(data=ex)
    prof = ex["kernel_profiles"][0]
    dims, B, act, dt = tuple(prof["dims"]), prof["batch"], prof["activation"], prof["dtype"]
    row = prof["kernel_entries"][0]
    cfg = pol.lookup_profile_kernel(dims=dims, batch=B, kind=row["kind"], M=row["shape"]["M"],
                                    K=row["shape"]["K"], activation=act, dtype=dt)
    assert cfg == TU.config_from_dict(row["config"])
    assert pol.lookup_profile_kernel(dims=dims, batch=B + 1, kind=row["kind"], M=row["shape"]["M"],
                                     K=row["shape"]["K"], activation=act, dtype=dt) is None
    g = ex["kernel_entries"][0]
    assert pol.lookup_kernel(kind=g["kind"], M=g["shape"]["M"], K=g["shape"]["K"], B=g["shape"]["B"],
                             activation=g["activation"], dtype=g["dtype"]) == TU.config_from_dict(g["config"])
    assert pol.profile_kernel_signature(dims=dims, batch=B, activation=act, dtype=dt) == prof["kernel_signature"]
    kw = dict(dims=dims, batch=B, activation=act, dtype=dt, kernel_sig=prof["kernel_signature"])
    best = ex["execution_entries"][0]["best"]
    assert pol.selected_grid_z(default=99, **kw) == best["grid_z_max_layers"]
    assert pol.selected_recompute_activation(default=not best["recompute_activation"], **kw) == \
        best["recompute_activation"]
    assert pol.selected_use_graph(default=not best["use_cuda_graph"], **kw) == best["use_cuda_graph"]
    # a different kernel table fingerprint does not resolve: defaults come back
    kw["kernel_sig"] = "0" * 20
    assert pol.selected_grid_z(default=99, **kw) == 99 and pol.selected_use_graph(default=False, **kw) is False


def test_policy_skips_malformed_rows_and_missing_files(tmp_path):
    pol = HP.HierarchicalPolicy(data={"kernel_entries": [{"kind": "prediction"}, 7],
                                      "kernel_profiles": [{"dims": "bad"}], "execution_entries": [{}]})
    assert pol.lookup_kernel(kind="prediction", M=1, K=1, B=1, activation="relu", dtype="float16") is None
    assert HP.load_hierarchical_policy(tmp_path / "none.json") is None
    with pytest.raises(ValueError):
        HP.HierarchicalPolicy(data=[1, 2])


GRIDZ = Path(__file__).parent / "golden" / "gridz_policy_excerpt.json"
RTX = dict(device_name="NVIDIA GeForce RTX 3060 Laptop GPU", capability=(8, 6), batch=128, activation="relu")


def test_gridz_key_format_reproduces_the_reference_keys():
    from lich_amd import gridz_tuning as GZ

    keys = set(json.loads(GRIDZ.read_text())["entries"])
    for dims in ((10, 64, 64, 64, 64, 784), (10,) + (64,) * 6 + (784,)):
        import torch
        assert GZ.make_policy_key(dims=dims, dtype=torch.float16, **RTX) in keys


def test_gridz_lookup_rules(tmp_path):
    from lich_amd import gridz_tuning as GZ

    d4, d6 = (10, 64, 64, 64, 64, 784), (10,) + (64,) * 6 + (784,)
    assert GZ.lookup_grid_z_cap(GRIDZ, dims=d4, dtype="float16", default=0, **RTX) == 3
    assert GZ.lookup_grid_z_cap(GRIDZ, dims=d6, dtype="float16", default=0, **RTX) == 2
    # another device, batch or dtype has no entry: the caller's default
    other = dict(RTX, device_name="AMD Instinct MI355X", capability=(9, 5))
    assert GZ.lookup_grid_z_cap(GRIDZ, dims=d4, dtype="float16", default=5, **other) == 5
    assert GZ.lookup_grid_z_cap(GRIDZ, dims=d4, dtype="bfloat16", default=4, **RTX) == 4
    assert GZ.lookup_grid_z_cap(tmp_path / "missing.json", dims=d4, dtype="float16", default=2, **RTX) == 2
    bad = tmp_path / "bad.json"
    bad.write_text(json.dumps({"entries": []}))
    with pytest.raises(ValueError):
        GZ.lookup_grid_z_cap(bad, dims=d4, dtype="float16", **RTX)


def test_table_reader_names_the_bad_row(tmp_path):
    p = tmp_path / "t.json"
    good = {"kind": "weight", "shape": {"M": 64, "K": 64, "B": 128}, "config": {"tile": 1}}
    for bad, needle in (({"kind": "weight", "config": {}}, "entry 1 lacks shape"),
                        ({"kind": "weight", "shape": {"M": 64, "K": "x", "B": 1}, "config": {}}, "entry 1 has no integer"),
                        ([1, 2], "entry 1 is a list")):
        p.write_text(json.dumps({"schema_version": 1, "entries": [good, bad]}))
        with pytest.raises(ValueError, match=needle):
            TU.TuningTable.from_json(p)
    # duplicates: the first matching entry wins, as a linear scan would give
    dup = dict(good, config={"tile": 2})
    p.write_text(json.dumps({"schema_version": 1, "entries": [good, dup]}))
    t = TU.TuningTable.from_json(p)
    assert t.lookup(kind="weight", M=64, K=64, B=128, activation="relu", dtype="float16").tile == 1
    p.write_text(json.dumps([good]))
    with pytest.raises(ValueError, match="JSON object"):
        TU.TuningTable.from_json(p)


def test_small_b_policy_skips_unusable_rows(tmp_path):
    from lich_amd.weight_update_specialization import SmallBWeightPolicy

    p = tmp_path / "p.json"
    rows = [{"M": 64, "K": 64, "B": 4, "backend": "outer", "activation": "tanh", "dtype": "float32"},
            {"M": 64, "K": 64, "B": 8, "backend": "cublas"}, {"K": 64, "B": 8}, "row", {"M": "a", "K": 1, "B": 1}]
    p.write_text(json.dumps({"entries": rows}))
    pol = SmallBWeightPolicy(p)
    assert len(pol.entries) == 1
    assert pol.backend(M=64, K=64, B=4, activation="tanh", dtype="torch.float32") == "outer"
    assert pol.backend(M=64, K=64, B=8, activation="relu", dtype="float16") == "gemm"
    p.write_text(json.dumps(rows))
    with pytest.raises(ValueError, match="JSON object"):
        SmallBWeightPolicy(p)
