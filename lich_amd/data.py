"""Offline datasets and the host-to-device batch pipeline of the training loop.

The reference trains on MNIST / FashionMNIST through torchvision with
``download=True`` (``scripts/train_mnist.py:42-52``) and moves each batch with
``prepare_batch`` (``src/ipc_tilelang/trainer.py:836-846``); pinned host input
with an asynchronous, double-buffered H2D pipeline is an open item of its
``README.md:171-172``.  Here:

* ``read_idx`` / ``load_dataset`` read the IDX files torchvision keeps under
  ``<root>/<name>/raw/`` (plain or ``.gz``) with numpy: nothing is fetched;
* ``synthetic_dataset`` is a seeded, MNIST-shaped stand-in with a learnable
  class structure (one prototype image per class plus noise) for machines
  without the files;
* ``BatchStager`` copies batches into two pinned host slots, issues their
  H2D copies on a side stream and lays them out on the device as the
  ``[features, B]`` input and ``[classes, B]`` one-hot target, so batch i+1
  crosses the bus while batch i trains.
"""
from __future__ import annotations

import gzip
from dataclasses import dataclass
from pathlib import Path
from typing import Iterator

import numpy as np
import torch

_IDX_DTYPES = {0x08: np.uint8, 0x09: np.int8, 0x0B: np.dtype(">i2"), 0x0C: np.dtype(">i4"),
               0x0D: np.dtype(">f4"), 0x0E: np.dtype(">f8")}

SPLIT_FILES = {
    True: ("train-images-idx3-ubyte", "train-labels-idx1-ubyte"),
    False: ("t10k-images-idx3-ubyte", "t10k-labels-idx1-ubyte"),
}


def read_idx(path: str | Path) -> np.ndarray:
    """An IDX file (the MNIST distribution format: two zero bytes, a type
    code, the number of dimensions, big-endian uint32 sizes, then the data),
    plain or gzip-compressed."""
    path = Path(path)
    raw = path.read_bytes()
    if raw[:2] == b"\x1f\x8b":
        raw = gzip.decompress(raw)
    if len(raw) < 4 or raw[0] != 0 or raw[1] != 0 or raw[2] not in _IDX_DTYPES:
        raise ValueError(f"{path}: not an IDX file")
    ndim = raw[3]
    head = 4 + 4 * ndim
    if len(raw) < head:
        raise ValueError(f"{path}: truncated IDX header")
    shape = tuple(int(v) for v in np.frombuffer(raw, dtype=">u4", count=ndim, offset=4))
    dtype = np.dtype(_IDX_DTYPES[raw[2]])
    count = int(np.prod(shape)) if shape else 1
    if len(raw) - head < count * dtype.itemsize:
        raise ValueError(f"{path}: {len(raw) - head} data bytes for shape {shape}")
    return np.frombuffer(raw, dtype=dtype, count=count, offset=head).reshape(shape).astype(dtype.newbyteorder("="))


def write_idx(path: str | Path, array: np.ndarray) -> None:
    """Writes ``array`` (uint8 or int32) as an IDX file (used by tests and to
    convert other sources)."""
    array = np.ascontiguousarray(array)
    codes = {np.dtype(np.uint8): 0x08, np.dtype(np.int32): 0x0C}
    if array.dtype not in codes:
        raise ValueError("write_idx supports uint8 and int32 arrays")
    head = bytes([0, 0, codes[array.dtype], array.ndim]) + np.asarray(array.shape, dtype=">u4").tobytes()
    data = array.astype(array.dtype.newbyteorder(">")).tobytes()
    blob = head + data
    path = Path(path)
    path.write_bytes(gzip.compress(blob) if path.suffix == ".gz" else blob)


def _find(root: Path, name: str, stem: str) -> Path:
    for folder in (root / name / "raw", root / name, root):
        for candidate in (folder / stem, folder / (stem + ".gz")):
            if candidate.is_file():
                return candidate
    raise FileNotFoundError(
        f"{stem}[.gz] not found under {root} (looked in {root / name / 'raw'}, {root / name}, {root}); "
        f"this build reads local files only: place the {name} IDX files there, or use synthetic_dataset()")


@dataclass
class ArrayDataset:
    """Images ``[N, H, W]`` (uint8, or float in [0, 1]) and int64 labels ``[N]``."""

    images: np.ndarray
    labels: np.ndarray
    num_classes: int = 10
    name: str = "dataset"

    def __post_init__(self) -> None:
        if len(self.images) != len(self.labels):
            raise ValueError("images and labels differ in length")

    def __len__(self) -> int:
        return int(len(self.labels))

    @property
    def features(self) -> int:
        return int(np.prod(self.images.shape[1:]))

    def subset(self, n: int) -> "ArrayDataset":
        n = min(int(n), len(self))
        return ArrayDataset(self.images[:n], self.labels[:n], self.num_classes, self.name)

    def batches(self, batch: int, *, shuffle: bool = True, seed: int = 0, epoch: int = 0,
                drop_last: bool = True) -> Iterator[tuple[torch.Tensor, torch.Tensor]]:
        """(images float32 ``[B, 1, H, W]`` scaled to [0, 1] as ``ToTensor``
        does, labels int64 ``[B]``), in a seeded order per epoch."""
        n = len(self)
        order = np.arange(n)
        if shuffle:
            order = np.random.default_rng([int(seed), int(epoch)]).permutation(n)
        stop = n - n % batch if drop_last else n
        for s in range(0, stop, batch):
            idx = order[s:s + batch]
            img = self.images[idx]
            img = img.astype(np.float32) / 255.0 if img.dtype == np.uint8 else img.astype(np.float32)
            yield (torch.from_numpy(img).unsqueeze(1), torch.from_numpy(self.labels[idx].astype(np.int64)))


def load_dataset(root: str | Path, name: str = "MNIST", *, train: bool = True, subset: int = 0) -> ArrayDataset:
    """MNIST / FashionMNIST from local IDX files (torchvision's layout); never downloads."""
    root = Path(root)
    img_stem, lab_stem = SPLIT_FILES[bool(train)]
    images = read_idx(_find(root, name, img_stem))
    labels = read_idx(_find(root, name, lab_stem)).astype(np.int64)
    if images.ndim != 3:
        raise ValueError(f"{name}: expected [N, H, W] images, got shape {images.shape}")
    ds = ArrayDataset(images, labels, 10, name)
    return ds.subset(subset) if subset else ds


def synthetic_dataset(n: int, *, seed: int = 0, num_classes: int = 10, shape: tuple[int, int] = (28, 28),
                      noise: float = 0.35) -> ArrayDataset:
    """Seeded MNIST-shaped data with a class structure: each class has a fixed
    random prototype in [0, 1]; a sample is its class prototype plus uniform
    noise, clipped to [0, 1] and quantised to uint8 like the real files."""
    rng = np.random.default_rng(int(seed))
    protos = rng.random((num_classes,) + tuple(shape), dtype=np.float32)
    labels = rng.integers(0, num_classes, size=int(n)).astype(np.int64)
    img = protos[labels] + noise * (rng.random((int(n),) + tuple(shape), dtype=np.float32) - 0.5)
    img = np.clip(np.rint(np.clip(img, 0.0, 1.0) * 255.0), 0, 255).astype(np.uint8)
    return ArrayDataset(img, labels, num_classes, f"synthetic(seed={seed})")


class BatchStager:
    """Double-buffered pinned-host -> device batch pipeline.

    ``put(images, labels)`` copies a CPU batch into the next pinned slot and
    enqueues its H2D copy on a side stream (default priority); ``get()``
    makes the caller's current stream wait for that copy, lays the batch out
    as ``x [features, B]`` and the one-hot ``y [classes, B]`` (the
    ``prepare_batch`` layout) and returns ``(x, y, labels)`` on the device.
    A slot is refilled only after the consumer stream has passed the point
    where the batch taken from it was used (an event recorded by ``get``), so
    up to two batches are in flight.
    """

    def __init__(self, batch: int, features: int, num_classes: int, *, device: torch.device,
                 dtype: torch.dtype = torch.float32, slots: int = 2):
        if not torch.cuda.is_available():
            raise RuntimeError("BatchStager needs a GPU")
        self.batch, self.features, self.num_classes = int(batch), int(features), int(num_classes)
        self.device, self.dtype = device, dtype
        self.copy_stream = torch.cuda.Stream(device=device)
        self._host_x = [torch.empty((self.batch, self.features), dtype=torch.float32, pin_memory=True)
                        for _ in range(slots)]
        self._host_l = [torch.empty((self.batch,), dtype=torch.int64, pin_memory=True) for _ in range(slots)]
        self._dev_x = [torch.empty((self.batch, self.features), dtype=torch.float32, device=device)
                       for _ in range(slots)]
        self._dev_l = [torch.empty((self.batch,), dtype=torch.int64, device=device) for _ in range(slots)]
        self._copied = [torch.cuda.Event() for _ in range(slots)]
        self._released = [None] * slots
        self._ready: list[int] = []
        self._next = 0

    def put(self, images: torch.Tensor, labels: torch.Tensor) -> None:
        if images.shape[0] != self.batch or labels.shape[0] != self.batch:
            raise ValueError(f"batch of {images.shape[0]} does not match the stager's {self.batch}")
        if len(self._ready) >= len(self._host_x):
            raise RuntimeError("every slot holds a batch that has not been taken")
        s = self._next
        self._next = (s + 1) % len(self._host_x)
        if self._released[s] is not None:
            # the host slot's previous H2D copy must have finished before refilling it
            self._copied[s].synchronize()
        self._host_x[s].copy_(images.reshape(self.batch, self.features))
        self._host_l[s].copy_(labels)
        with torch.cuda.stream(self.copy_stream):
            if self._released[s] is not None:
                self.copy_stream.wait_event(self._released[s])
            self._dev_x[s].copy_(self._host_x[s], non_blocking=True)
            self._dev_l[s].copy_(self._host_l[s], non_blocking=True)
            self._copied[s].record(self.copy_stream)
        self._ready.append(s)

    def get(self) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        if not self._ready:
            raise RuntimeError("no staged batch")
        s = self._ready.pop(0)
        cur = torch.cuda.current_stream(self.device)
        cur.wait_event(self._copied[s])
        x = self._dev_x[s].T.to(dtype=self.dtype).contiguous()
        y = torch.nn.functional.one_hot(self._dev_l[s], self.num_classes).to(dtype=self.dtype).T.contiguous()
        labels = self._dev_l[s].clone()
        ev = torch.cuda.Event()
        ev.record(cur)
        self._released[s] = ev
        return x, y, labels
