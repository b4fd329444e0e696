"""torch.utils.data-style loading for oxitorch_amd (python/oxitorch/utils/data.py).

Same API as the reference module. Two paths behind one `DataLoader`:

- **Device path** for datasets that expose `tensors` (column tensors sharing
  dim 0, e.g. `TensorDataset`) with the default collation and no custom
  sampler: `_native.DataLoader` keeps the columns in HBM for the loader's
  lifetime, uploads each epoch's row order once, and gathers every batch on
  the device, one launch for all columns. Shuffled orders are NumPy's
  `RandomState(seed + epoch).permutation(n)`, as in the reference's native
  loader. The only host work is each epoch's permutation; `num_workers`
  host threads (at least one) compute the coming epochs' orders ahead.
- **Generic path** for any other `Dataset` / `IterableDataset`: items are
  fetched per index (through a thread pool when `num_workers > 1`) and
  collated with `default_collate`; the collated batch is uploaded through the
  library's pinned staging ring without waiting for the device.

As in the reference, labels are f32 tensors.
"""

import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np

from oxitorch_amd import _native

__all__ = [
    "DataLoader",
    "Dataset",
    "IterableDataset",
    "RandomSampler",
    "SequentialSampler",
    "Subset",
    "TensorDataset",
    "default_collate",
]


class Dataset:
    """Map-style dataset: `__getitem__` and `__len__`."""

    def __getitem__(self, index):
        raise NotImplementedError

    def __len__(self):
        raise NotImplementedError


class IterableDataset(Dataset):
    """Stream-style dataset: `__iter__`."""

    def __iter__(self):
        raise NotImplementedError


class TensorDataset(Dataset):
    """Rows of several tensors that share dim 0."""

    def __init__(self, *tensors):
        rows = tensors[0].shape[0]
        for k, t in enumerate(tensors):
            if t.shape[0] != rows:
                raise ValueError(f"tensor {k} has {t.shape[0]} rows, expected {rows}")
        self.tensors = tensors

    def __getitem__(self, index):
        return tuple(t[index] for t in self.tensors)

    def __len__(self):
        return self.tensors[0].shape[0]


class Subset(Dataset):
    """The rows `indices` of another dataset, fetched per item."""

    def __init__(self, dataset, indices):
        self.dataset = dataset
        self.indices = list(indices)

    def __getitem__(self, index):
        return self.dataset[self.indices[index]]

    def __len__(self):
        return len(self.indices)


class Sampler:
    """An index stream."""

    def __iter__(self):
        raise NotImplementedError

    def __len__(self):
        raise NotImplementedError


class SequentialSampler(Sampler):
    def __init__(self, data_source):
        self.data_source = data_source

    def __iter__(self):
        return iter(range(len(self.data_source)))

    def __len__(self):
        return len(self.data_source)


class RandomSampler(Sampler):
    """A permutation per pass; with `seed`, pass k uses RandomState(seed + k)."""

    def __init__(self, data_source, seed=None):
        self.data_source = data_source
        self.seed = seed
        self._epoch = 0

    def __iter__(self):
        n = len(self.data_source)
        if self.seed is None:
            order = np.random.permutation(n)
        else:
            order = np.random.RandomState(self.seed + self._epoch).permutation(n)
            self._epoch += 1
        return (int(i) for i in order)

    def __len__(self):
        return len(self.data_source)


def _stack_f32(arrays):
    return np.ascontiguousarray(np.stack([np.asarray(a, dtype=np.float32) for a in arrays]))


def default_collate(items):
    """Batches fetched items: tuples field by field, tensors and numpy arrays
    stacked into an f32 tensor (tensors keep `requires_grad` when all have
    it), Python numbers into an f32 vector."""
    if not items:
        raise ValueError("cannot collate an empty item list")
    head = items[0]
    if isinstance(head, (tuple, list)):
        return tuple(default_collate([it[k] for it in items]) for k in range(len(head)))
    if isinstance(head, np.ndarray):
        return _native.from_numpy(_stack_f32(items))
    if hasattr(head, "shape") and hasattr(head, "numpy"):
        rg = all(bool(getattr(it, "requires_grad", False)) for it in items)
        return _native.from_numpy(_stack_f32([it.detach().numpy() for it in items]), rg)
    if isinstance(head, (int, float)):
        return _native.from_numpy(np.ascontiguousarray(np.asarray(items, dtype=np.float32)))
    raise TypeError(f"default_collate cannot handle items of type {type(head)!r}")


class DataLoader:
    """Batches a dataset with torch's constructor surface. Each `__iter__`
    is one epoch; seeded shuffles are reproducible epoch by epoch."""

    def __init__(self, dataset, batch_size=1, shuffle=False, sampler=None, batch_sampler=None, num_workers=0,
                 collate_fn=default_collate, drop_last=False, seed=None):
        if batch_size < 1:
            raise ValueError("batch_size must be >= 1")
        self.dataset = dataset
        self.batch_size = batch_size
        self.shuffle = shuffle
        self.sampler = sampler
        self.batch_sampler = batch_sampler
        self.num_workers = num_workers
        self.collate_fn = collate_fn
        self.drop_last = drop_last
        self.seed = seed
        # an unseeded loader still varies by run: a random base drawn once
        self._auto_seed = int.from_bytes(os.urandom(4), "little")
        self._epoch = 0
        self._device_loader = None

    def __len__(self):
        if self.batch_sampler is not None:
            return len(self.batch_sampler)
        if isinstance(self.dataset, IterableDataset):
            raise TypeError("IterableDataset has no length; len(DataLoader) is undefined")
        n = len(self.dataset)
        return n // self.batch_size if self.drop_last else -(-n // self.batch_size)

    def _device_path(self):
        """The device loader for tensor-column datasets, built once (its
        columns are uploaded to HBM a single time), or None."""
        if self.sampler is not None or self.batch_sampler is not None or self.collate_fn is not default_collate:
            return None
        if getattr(self.dataset, "native_parts", None) is not None:
            return None  # datasets with native transforms take the per-item path here
        tensors = getattr(self.dataset, "tensors", None)
        if tensors is None:
            return None
        if self._device_loader is None:
            cols = [t if isinstance(t, _native.Tensor) else _native.from_numpy(np.ascontiguousarray(t, np.float32))
                    for t in tensors]
            base = self.seed if self.seed is not None else self._auto_seed
            self._device_loader = _native.DataLoader(cols, batch_size=self.batch_size, shuffle=self.shuffle,
                                                     drop_last=self.drop_last, seed=base,
                                                     num_workers=self.num_workers)
        return self._device_loader

    def __iter__(self):
        epoch = self._epoch
        self._epoch += 1
        dev = self._device_path()
        if dev is not None:
            # the device loader's own epoch counter follows this one: the
            # order of pass k is RandomState(seed + k).permutation(n)
            yield from iter(dev)
            return
        if self.batch_sampler is not None:
            for batch in self.batch_sampler:
                yield self._collate(list(batch))
            return
        if isinstance(self.dataset, IterableDataset):
            yield from self._stream()
            return
        if self.sampler is not None:
            order = iter(self.sampler)
        elif self.shuffle:
            order = iter(RandomSampler(self.dataset, seed=None if self.seed is None else self.seed + epoch))
        else:
            order = iter(SequentialSampler(self.dataset))
        batch = []
        for i in order:
            batch.append(i)
            if len(batch) == self.batch_size:
                yield self._collate(batch)
                batch = []
        if batch and not self.drop_last:
            yield self._collate(batch)

    def _stream(self):
        items = []
        for item in self.dataset:
            items.append(item)
            if len(items) == self.batch_size:
                yield self.collate_fn(items)
                items = []
        if items and not self.drop_last:
            yield self.collate_fn(items)

    def _collate(self, batch):
        if self.num_workers > 1 and len(batch) > 1:
            with ThreadPoolExecutor(max_workers=self.num_workers) as pool:
                items = list(pool.map(self.dataset.__getitem__, batch))
        else:
            items = [self.dataset[i] for i in batch]
        return self.collate_fn(items)
