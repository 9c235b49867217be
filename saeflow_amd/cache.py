"""Activation caching with on-the-fly SAE encoding: the caller of the hot path that feeds it
model activations and stores its CSR output (reference saeflow/cache.py).

The API (cache_activations, ActivationReader) and the on-disk format are the reference's,
so a cache written by either side reads on the other (cache.py:1-13):

    manifest.json                                   {"config", "hooks", "shards"}
    <hook>/<shard:05d>.npy                          dense activations [rows, d]
    <hook>/<shard:05d>.{indptr,indices,values}.npy  CSR features [rows, d_sae] (encoded hooks)

Rows are token positions in sequence-major order, a shard holds `batches_per_shard`
forward batches, bfloat16 arrays hold the raw 16-bit patterns (numpy has no bfloat16; the
manifest names the dtype), and a shard's files are fsynced and renamed into place before the
manifest lists it, so an interrupted run keeps whole shards only and a rerun with the same
arguments continues at the first missing shard.

What differs is how the work is overlapped on the GPU box (the reference runs forward,
encode, copy and write one after the other; its roadmap, README.md:234-235, asks for the
copy overlap):
  - encoded hooks go through saeflow_amd.encode_sparse, whose row-candidate encode never
    forms the dense [rows, d_sae] features;
  - results leave the GPU on a copy stream into pinned host memory, so the next batch's
    forward pass runs while the last one is copied;
  - a writer thread waits for a finished shard's copies, writes it piece by piece (the
    batches' CSR pieces with moved indptr offsets, dense rows as they are, after numpy's own
    .npy header: the bytes of np.save of the joined array, without forming it; numpy on one
    thread, as torch's host thread pool would take cores from the caller's kernel launches),
    fsyncs it and then lists it in the
    manifest, in shard order, while the GPU already works on the next shard; the caller
    never waits at a shard boundary.
"""

import bisect
import functools
import json
import os
import queue
import threading
from pathlib import Path

import numpy as np
import torch

_DTYPE_NAMES = {torch.float32: "float32", torch.float16: "float16", torch.bfloat16: "bfloat16"}
_CSR_FILES = ("indptr", "indices", "values")


# ----------------------------------------------------------------------------- format
def _as_stored(t):
    """Host tensor -> the numpy array the format stores (bfloat16 as its int16 bit pattern)."""
    t = t.detach().contiguous().cpu()
    return t.view(torch.int16).numpy() if t.dtype == torch.bfloat16 else t.numpy()


def _as_tensor(a, dtype):
    """Stored numpy array (possibly a read-only memory map) -> torch tensor of `dtype`."""
    t = torch.from_numpy(np.ascontiguousarray(a).copy())
    return t.view(torch.bfloat16) if dtype == torch.bfloat16 else t


def _write_durably(path, payload):
    """Write `payload(fh)` to a sibling temporary, fsync it, then rename it over `path`."""
    tmp = path.parent / f".{path.name}.partial.tmp"
    with open(tmp, "wb") as fh:
        payload(fh)
        fh.flush()
        os.fsync(fh.fileno())
    os.replace(tmp, path)


def _shard_file(root, hook, shard, part=None):
    return Path(root) / hook / (f"{shard:05d}.npy" if part is None else f"{shard:05d}.{part}.npy")


def _join_csr(pieces):
    """Row-wise concatenation of CSR pieces [(indptr, indices, values)] on the host."""
    ends = np.cumsum([int(p[0][-1]) for p in pieces])
    starts = np.concatenate([[0], ends[:-1]]).astype(np.int64)
    indptr = torch.cat([torch.zeros(1, dtype=torch.int64)] + [p[0][1:].cpu() + int(s) for p, s in zip(pieces, starts)])
    return indptr, torch.cat([p[1].cpu() for p in pieces]), torch.cat([p[2].cpu() for p in pieces])


def _blocks_needed(hook_names):
    """Number of transformer blocks the deepest requested hook needs, if every hook is a
    `blocks.<i>.` hook (the forward stops there, cache.py:64-67); None otherwise."""
    depth = 0
    for h in hook_names:
        head, _, rest = h.partition(".")
        idx, _, _ = rest.partition(".")
        if head != "blocks" or not idx.isdigit():
            return None
        depth = max(depth, int(idx) + 1)
    return depth


# ----------------------------------------------------------------------------- writing
class _Staging:
    """Device -> host copies of one shard, on a side stream into pinned host buffers."""

    def __init__(self):
        self.stream = None
        self.copies = []

    def to_host(self, t):
        t = t.detach().contiguous()
        if not t.is_cuda:
            return t
        if self.stream is None:
            self.stream = torch.cuda.Stream(t.device)  # default priority
        host = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
        produced = torch.cuda.Event()
        produced.record(torch.cuda.current_stream(t.device))
        with torch.cuda.stream(self.stream):
            self.stream.wait_event(produced)
            host.copy_(t, non_blocking=True)
            landed = torch.cuda.Event()
            landed.record(self.stream)
        t.record_stream(self.stream)  # the caching allocator keeps t's memory until then
        self.copies.append(landed)
        return host

    def take(self):
        """The events of the copies issued since the last call (the shard's), handed over."""
        copies, self.copies = self.copies, []
        return copies


def _save_rows(fh, pieces):
    """Writes what np.save(fh, np.concatenate(pieces)) writes (the .npy format, version 1.0:
    numpy's own header for the joined shape, then the rows in C order) without forming the
    joined array: each piece's buffer goes straight to the file, and the GIL is released
    while it is written."""
    first = pieces[0]
    shape = (sum(int(p.shape[0]) for p in pieces),) + tuple(first.shape[1:])
    np.lib.format.write_array_header_1_0(fh, {"descr": np.lib.format.dtype_to_descr(first.dtype),
                                              "fortran_order": False, "shape": shape})
    for p in pieces:
        if p.size:
            fh.write(np.ascontiguousarray(p).data)


def _shard_arrays(out_dir, shard, held, csr_hooks):
    """The files of a finished shard as lists of stored numpy pieces, one list per file, to be
    written one after the other: per hook, the row-wise concatenation of its batches (CSR
    pieces with their indptr offsets moved, dense rows as they are). Plain numpy and no joined
    copies: this runs beside the caller, whose kernel launches must not wait for cores or the
    GIL."""
    files = []
    for h, pieces in held.items():
        parts = [[_as_stored(t) for t in (p if isinstance(p, tuple) else (p,))] for p in pieces]
        if h in csr_hooks:
            ends = np.cumsum([int(p[0][-1]) for p in parts])
            starts = np.concatenate([[0], ends[:-1]]).astype(np.int64)
            indptr = [np.zeros(1, np.int64)] + [p[0][1:] + s for p, s in zip(parts, starts)]
            for part, rows in zip(_CSR_FILES, (indptr, [p[1] for p in parts], [p[2] for p in parts])):
                files.append((_shard_file(out_dir, h, shard, part), rows))
        else:
            files.append((_shard_file(out_dir, h, shard), [p[0] for p in parts]))
    return files


class _Writer(threading.Thread):
    """Writes finished shards in order, each followed by its manifest entry; a failure is
    re-raised to the caller at the next hand-over or at close(). A job is (events of the
    shard's device -> host copies, a function assembling its files, hook metadata, manifest
    entry)."""

    def __init__(self, manifest, manifest_path):
        super().__init__(daemon=True)
        self.manifest, self.manifest_path = manifest, manifest_path
        self.inbox = queue.Queue(maxsize=2)  # at most two finished shards wait in host memory
        self.failure = None
        self.start()

    def run(self):
        for job in iter(self.inbox.get, None):
            if self.failure is not None:
                continue
            try:
                copies, build, hook_meta, entry = job
                for ev in copies:
                    ev.synchronize()  # the shard's device -> host copies; blocks without the GIL
                for path, rows in build():
                    _write_durably(path, lambda fh, rows=rows: _save_rows(fh, rows))
                self.manifest["hooks"].update(hook_meta)
                self.manifest["shards"].append(entry)
                text = json.dumps(self.manifest, indent=2).encode()
                _write_durably(self.manifest_path, lambda fh: fh.write(text))
            except BaseException as e:
                self.failure = e

    def hand_over(self, job):
        if self.failure is not None:
            raise self.failure
        self.inbox.put(job)

    def close(self):
        self.inbox.put(None)
        self.join()
        if self.failure is not None:
            raise self.failure


@torch.inference_mode()
def cache_activations(model, tokens, hook_names, out_dir, *, batch_size=8, batches_per_shard=32,
                      dtype=torch.float32, encoders=None):
    """Run `model` over `tokens` [n_seqs, seq_len] and cache the activations at `hook_names`
    (reference cache.py:70-130: same arguments, result and errors).

    model: anything with a TransformerLens-style run_with_cache(tokens, names_filter=,
      stop_at_layer=, return_type=) and parameters().
    encoders: optional {hook_name: sae}; those hooks are SAE-encoded on the fly on the GPU
      and stored as CSR feature activations instead of dense ones.
    A second call with identical arguments after an interruption picks up at the first shard
    the manifest does not list. The return value is the cache directory (a Path).
    """
    out_dir, hook_names, encoders = Path(out_dir), list(hook_names), dict(encoders or {})
    if dtype not in _DTYPE_NAMES:
        raise ValueError(f"cache dtype must be one of {list(_DTYPE_NAMES)}, got {dtype}")
    stray = sorted(set(encoders) - set(hook_names))
    if stray:
        raise ValueError(f"encoders given for hooks not being cached: {stray}")
    if encoders:
        from .ops import encode_sparse

    config = {"hook_names": hook_names, "n_seqs": len(tokens), "seq_len": int(tokens.shape[1]),
              "batch_size": batch_size, "batches_per_shard": batches_per_shard, "dtype": _DTYPE_NAMES[dtype],
              "encoded": sorted(encoders)}
    manifest_path = out_dir / "manifest.json"
    manifest = {"config": config, "hooks": {}, "shards": []}
    if manifest_path.exists():
        manifest = json.loads(manifest_path.read_text())
        if manifest["config"] != config:
            raise ValueError(f"{out_dir} holds a cache with a different config: {manifest['config']}")
    for h in hook_names:
        (out_dir / h).mkdir(parents=True, exist_ok=True)

    device = next(iter(model.parameters())).device
    if device.type == "cuda" and tokens.device.type == "cpu" and not tokens.is_pinned():
        # uploads from pinned memory are asynchronous: the next batch's tokens go up while the
        # GPU still works on this one (a pageable upload first waits for the stream to drain)
        tokens = tokens.contiguous().pin_memory()
    depth = _blocks_needed(hook_names)
    per_shard = batch_size * batches_per_shard
    shard_starts = list(range(0, len(tokens), per_shard))
    writer = _Writer(manifest, manifest_path)
    staging = _Staging()
    try:
        for shard in range(len(manifest["shards"]), len(shard_starts)):
            lo = shard_starts[shard]
            hi = min(lo + per_shard, len(tokens))
            held = {h: [] for h in hook_names}
            for b0 in range(lo, hi, batch_size):
                batch = tokens[b0:min(b0 + batch_size, hi)].to(device, non_blocking=True)
                _, acts = model.run_with_cache(batch, names_filter=hook_names, stop_at_layer=depth, return_type=None)
                for h in hook_names:
                    rows = acts[h].reshape(acts[h].shape[0] * acts[h].shape[1], -1)  # per-head hooks concatenated
                    sae = encoders.get(h)
                    if sae is None:
                        held[h].append(staging.to_host(rows.to(dtype)))
                    else:
                        csr = encode_sparse(sae, rows.to(sae.W_enc.device, sae.W_enc.dtype))
                        held[h].append((staging.to_host(csr[0]), staging.to_host(csr[1]),
                                        staging.to_host(csr[2].to(dtype))))
            hook_meta = {h: {"format": "csr", "d": int(encoders[h].W_enc.shape[1])} if h in encoders
                         else {"format": "dense", "d": int(held[h][0].shape[1])} for h in hook_names}
            # the shard is assembled (CSR pieces joined, dense rows stacked) by the writer thread
            build = functools.partial(_shard_arrays, out_dir, shard, held, frozenset(encoders))
            writer.hand_over((staging.take(), build, hook_meta, {"n_seqs": hi - lo, "n_rows": (hi - lo) * config["seq_len"]}))
    finally:
        writer.close()  # shards already handed over are written even when the run fails
    return out_dir


# ----------------------------------------------------------------------------- reading
class ActivationReader:
    """Streams a cache written by cache_activations back in batches (reference
    cache.py:133-190). Shards are memory-mapped; a batch may span shards."""

    def __init__(self, path):
        self.path = Path(path)
        self.manifest = json.loads((self.path / "manifest.json").read_text())
        self.dtype = {v: k for k, v in _DTYPE_NAMES.items()}[self.manifest["config"]["dtype"]]
        rows = [s["n_rows"] for s in self.manifest["shards"]]
        self._first_row = np.concatenate([[0], np.cumsum(rows)]).astype(np.int64).tolist()

    @property
    def hook_names(self):
        return self.manifest["config"]["hook_names"]

    def n_rows(self):
        return self._first_row[-1]

    def _sparse(self, hook):
        return self.manifest["hooks"][hook]["format"] == "csr"

    def _load(self, hook, shard):
        if self._sparse(hook):
            return tuple(np.load(_shard_file(self.path, hook, shard, p), mmap_mode="r") for p in _CSR_FILES)
        return np.load(_shard_file(self.path, hook, shard), mmap_mode="r")

    def _piece(self, hook, arrays, a, b):
        """Rows [a, b) of one shard."""
        if not self._sparse(hook):
            return _as_tensor(arrays[a:b], self.dtype)
        indptr, indices, values = arrays
        lo, hi = int(indptr[a]), int(indptr[b])
        return (torch.from_numpy(np.asarray(indptr[a:b + 1], dtype=np.int64) - lo),
                _as_tensor(indices[lo:hi], torch.int32), _as_tensor(values[lo:hi], self.dtype))

    def iter_batches(self, hook, batch_size):
        """Yield `batch_size`-row batches in cache order (the last may be short). Dense hooks
        yield [rows, d] tensors; encoded hooks yield CSR (indptr, indices, values) tuples, which
        decode_sparse takes once they are on the GPU."""
        total, opened = self.n_rows(), {}
        for start in range(0, total, batch_size):
            stop = min(start + batch_size, total)
            pieces, r = [], start
            while r < stop:
                shard = bisect.bisect_right(self._first_row, r) - 1
                if shard not in opened:
                    opened = {shard: self._load(hook, shard)}  # keep only the current shard's maps
                base = self._first_row[shard]
                end = min(stop, self._first_row[shard + 1])
                pieces.append(self._piece(hook, opened[shard], r - base, end - base))
                r = end
            yield _join_csr(pieces) if self._sparse(hook) else torch.cat(pieces)
