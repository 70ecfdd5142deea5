"""Offline dataset reader, synthetic data, CLI wiring and the telemetry guard (no GPU)."""
import gzip
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from lich_amd import data as D
from lich_amd import telemetry as T
from lich_amd import train as TR

FIXTURE = Path(__file__).parent / "data" / "amd_smi_metric_tpcu.json"


@pytest.mark.parametrize("suffix", ["", ".gz"])
def test_idx_round_trip_and_torchvision_layout(tmp_path, suffix):
    rng = np.random.default_rng(1)
    images = rng.integers(0, 256, size=(37, 28, 28), dtype=np.uint8)
    labels = rng.integers(0, 10, size=37).astype(np.uint8)
    raw = tmp_path / "MNIST" / "raw"
    raw.mkdir(parents=True)
    D.write_idx(raw / ("train-images-idx3-ubyte" + suffix), images)
    D.write_idx(raw / ("train-labels-idx1-ubyte" + suffix), labels)
    # the header is the published IDX layout: 0, 0, type 0x08, 3 dims, big-endian sizes
    blob = (raw / ("train-images-idx3-ubyte" + suffix)).read_bytes()
    if suffix:
        blob = gzip.decompress(blob)
    assert blob[:4] == bytes([0, 0, 8, 3]) and blob[4:16] == (37).to_bytes(4, "big") + (28).to_bytes(4, "big") * 2
    ds = D.load_dataset(tmp_path, "MNIST", train=True)
    assert np.array_equal(ds.images, images) and np.array_equal(ds.labels, labels.astype(np.int64))
    assert len(D.load_dataset(tmp_path, "MNIST", subset=10)) == 10


def test_missing_dataset_names_the_paths_and_never_downloads(tmp_path):
    with pytest.raises(FileNotFoundError, match="local files only"):
        D.load_dataset(tmp_path, "FashionMNIST")


def test_idx_rejects_garbage(tmp_path):
    p = tmp_path / "x"
    p.write_bytes(b"\x01\x02\x03\x04")
    with pytest.raises(ValueError, match="not an IDX"):
        D.read_idx(p)
    D.write_idx(p, np.zeros((4, 3), np.uint8))
    p.write_bytes(p.read_bytes()[:-2])
    with pytest.raises(ValueError, match="data bytes"):
        D.read_idx(p)


def test_synthetic_dataset_is_seeded_and_class_structured():
    a, b = D.synthetic_dataset(500, seed=3), D.synthetic_dataset(500, seed=3)
    assert np.array_equal(a.images, b.images) and np.array_equal(a.labels, b.labels)
    assert a.images.dtype == np.uint8 and a.images.shape == (500, 28, 28) and a.features == 784
    # nearest class mean recovers the labels: the data is learnable
    x = a.images.reshape(500, -1).astype(np.float64)
    means = np.stack([x[a.labels == c].mean(0) for c in range(10)])
    pred = ((x[:, None, :] - means[None]) ** 2).sum(-1).argmin(1)
    assert (pred == a.labels).mean() > 0.95


def test_batches_scale_like_totensor_and_cover_the_epoch():
    ds = D.synthetic_dataset(100, seed=0)
    got = list(ds.batches(32, shuffle=True, seed=5, epoch=1))
    assert len(got) == 3 and all(img.shape == (32, 1, 28, 28) for img, _ in got)
    img, lab = got[0]
    order = np.random.default_rng([5, 1]).permutation(100)[:32]
    assert torch.equal(img, torch.from_numpy(ds.images[order].astype(np.float32) / 255.0).unsqueeze(1))
    assert torch.equal(lab, torch.from_numpy(ds.labels[order]))
    seen = np.concatenate([l.numpy() for _, l in ds.batches(10, shuffle=False, drop_last=False)])
    assert np.array_equal(seen, ds.labels)


def test_train_cli_defaults_follow_the_reference_script():
    a = TR.parse_args([])
    assert (a.hidden, a.depth, a.batch, a.epochs, a.steps, a.alpha, a.gamma, a.activation) == \
        (64, 2, 128, 5, 4, 1e-4, 0.5, "relu")
    a = TR.parse_args(["--synthetic", "1000", "--graph", "--dataset", "FashionMNIST"])
    assert a.synthetic == 1000 and a.graph and a.dataset == "FashionMNIST"


def test_parse_amd_smi_fixture():
    t = T.parse_amd_smi_metric(json.loads(FIXTURE.read_text()))
    assert t.temperature_c == 46.0 and t.temperature_mem_c == 34.0 and t.power_w == 241.0
    assert t.clock_mem_mhz == 2000.0 and t.clock_gfx_max_mhz == 2400.0
    assert t.clock_gfx_mhz == pytest.approx((113 + 114 + 94 + 95 + 94 + 95 + 96 + 96) / 8)
    assert t.util_gpu_pct == 0.0 and t.util_mem_pct == 0.0
    assert t.throttle_status == "N/A" and not (t.thermal_throttle or t.power_limited or t.hardware_slowdown)
    # the fixture is amd-smi's {"gpu_data": [...]}; the bare per-GPU record and a list of them parse alike
    inner = json.loads(FIXTURE.read_text())["gpu_data"][0]
    assert T.parse_amd_smi_metric(inner) == t and T.parse_amd_smi_metric([inner]) == t
    assert "temp=46.0C" in T.ThermalGuard.format_status(t)


def test_thermal_guard_hysteresis_and_rate_limit():
    temps = iter([97.0, 96.0, 92.0, 90.0, 99.0])
    calls = []

    def reader():
        calls.append(1)
        return T.Telemetry(next(temps), None, None, None, None, None)

    g = T.ThermalGuard(max_temp_c=95.0, poll_s=0.0, telemetry_interval_s=3600.0, reader=reader)
    t = g.wait_until_safe()
    # paused at 97, kept pausing at 96 and 92 (resume at 91), resumed at 90
    assert t.temperature_c == 90.0 and g.pauses == 1 and len(calls) == 4
    assert g.wait_until_safe().temperature_c == 90.0 and len(calls) == 4  # cached sample, no query
    throttled = T.Telemetry(80.0, None, None, None, None, None, throttle_status="THERMAL")
    g2 = T.ThermalGuard(reader=lambda: throttled, poll_s=0.0)
    with pytest.raises(RuntimeError, match="thermal throttle"):
        g2.assert_no_thermal_throttle()
    assert g2.wait_until_safe(max_wait_s=0.0).thermal_throttle


def test_read_telemetry_never_raises():
    t = T.read_telemetry(0, timeout_s=20.0)
    assert isinstance(t, T.Telemetry)
