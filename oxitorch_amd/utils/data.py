"""Batches that land on the device: the input-pipeline row of this build.

A dataset of column tensors that share their first dim (`TensorDataset`) is
uploaded to HBM once, when its loader is made. Every batch is then one
device gather of all columns at the batch's rows (`_native.DataLoader`,
oxi_batch_gather). The rows come in order, or shuffled per epoch as
NumPy's `RandomState(seed + epoch).permutation(n)`, the order the reference's
native loader draws (crates/oxi-data/src/batch.rs:223-292, rng.rs); the host
computes coming epochs' orders on `num_workers` threads, and that is all the
host does per epoch.

The constructor keeps the reference's signature
(python/oxitorch/utils/data.py:167-201). Its per-item path (any map-style or
iterable dataset fetched item by item, samplers, custom collation) stays on
the host in the reference and is not part of this device build: those
arguments raise NotImplementedError. Batches are leaf tensors without
gradient, f32 like the reference's.

Every public name of the reference module (data.py:31-40) is here, so code
written against it imports unchanged: `Dataset` and `IterableDataset` are the
base classes a user dataset derives from; the per-item pieces (`Subset`, the
samplers, `default_collate`) raise NotImplementedError when used.
"""

import os

import numpy as np

from oxitorch_amd import _native

__all__ = ["DataLoader", "Dataset", "IterableDataset", "RandomSampler", "SequentialSampler", "Subset",
           "TensorDataset", "default_collate"]

_PER_ITEM = ("runs item by item on the host in the reference; this build's loader gathers whole batches of "
             "column tensors (TensorDataset) on the device")


class Dataset:
    """Base of map-style datasets: a subclass gives `__getitem__` and `__len__`."""

    def __getitem__(self, index):
        raise NotImplementedError(f"{type(self).__name__} does not define __getitem__")

    def __len__(self):
        raise NotImplementedError(f"{type(self).__name__} does not define __len__")


class IterableDataset(Dataset):
    """Base of stream-style datasets: a subclass gives `__iter__`."""

    def __iter__(self):
        raise NotImplementedError(f"{type(self).__name__} does not define __iter__")


class _PerItem:
    """A per-item piece of the reference's host loader: refused when made."""

    def __init__(self, *args, **kwargs):
        raise NotImplementedError(f"{type(self).__name__} {_PER_ITEM}")


class Subset(_PerItem, Dataset):
    """The reference's index view of a dataset (not built: per-item)."""


class Sampler(_PerItem):
    """The reference's index-stream base (not built: per-item)."""


class SequentialSampler(Sampler):
    """The reference's in-order index stream (not built: per-item)."""


class RandomSampler(Sampler):
    """The reference's shuffled index stream (not built: per-item)."""


def default_collate(items):
    """The reference's item collation (not built: per-item)."""
    raise NotImplementedError(f"default_collate {_PER_ITEM}")


def _on_device(column):
    if isinstance(column, _native.Tensor):
        return column
    return _native.from_numpy(np.ascontiguousarray(column, dtype=np.float32))


class TensorDataset(Dataset):
    """Column tensors of equal length; item i is the tuple of their i-th rows."""

    def __init__(self, *tensors):
        lengths = [t.shape[0] for t in tensors]
        for k, rows in enumerate(lengths):
            if rows != lengths[0]:
                raise ValueError(f"tensor {k} has {rows} rows, expected {lengths[0]}")
        self.tensors = tensors

    def __len__(self):
        return self.tensors[0].shape[0]

    def __getitem__(self, index):
        return tuple(column[index] for column in self.tensors)


class DataLoader:
    """Device batches of a column dataset; each `iter()` is one epoch."""

    def __init__(self, dataset, batch_size=1, shuffle=False, sampler=None, batch_sampler=None, num_workers=0,
                 collate_fn=None, drop_last=False, seed=None):
        if batch_size < 1:
            raise ValueError("batch_size must be >= 1")
        unsupported = [name for name, v in (("sampler", sampler), ("batch_sampler", batch_sampler),
                                            ("collate_fn", collate_fn)) if v is not None]
        if unsupported:
            raise NotImplementedError(
                f"DataLoader({', '.join(unsupported)}=...): custom sampling and collation run item by item on the "
                "host; this build's loader gathers whole batches of column tensors on the device")
        columns = getattr(dataset, "tensors", None)
        if columns is None:
            raise NotImplementedError(
                f"DataLoader over {type(dataset).__name__}: only datasets of column tensors (TensorDataset) have a "
                "device path; per-item datasets are outside this build")
        self.dataset = dataset
        self.batch_size = batch_size
        self.shuffle = shuffle
        self.drop_last = drop_last
        self.num_workers = num_workers
        # an unseeded loader draws one random base, so runs differ while the
        # epochs of one run stay reproducible; `seed` fixes it
        self.seed = seed if seed is not None else int.from_bytes(os.urandom(4), "little")
        self._batches = _native.DataLoader([_on_device(c) for c in columns], batch_size=batch_size,
                                           shuffle=shuffle, drop_last=drop_last, seed=self.seed,
                                           num_workers=num_workers)

    def __len__(self):
        rows = len(self.dataset)
        full, rest = divmod(rows, self.batch_size)
        return full + (1 if rest and not self.drop_last else 0)

    def __iter__(self):
        return iter(self._batches)
