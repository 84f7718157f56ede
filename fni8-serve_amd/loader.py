"""Checkpoint loading over the `.fni8` container.

Same functions, arguments and errors as fni8serve/loader.py:19-69:
`load_fni8_checkpoint` (all tensors, an explicit name list, or one shard of
the shard index: "pp:<stage>" or an expert key), `load_fni8_state_dict`
(unwraps "raw" tensors to plain tensors, the form the layer builders take) and
`checkpoint_info` (header summary, no tensor data read).  Only the pages of the
requested tensors are touched, since the container is memory-mapped.
"""
from __future__ import annotations

from .container import FQReader
from .qtensor import QTensor


def _shard_names(index: dict, shard: str) -> list[str]:
    experts = index.get("experts", {})
    if shard in experts:
        return list(experts[shard])
    if shard.startswith("pp:"):
        return list(index["pp_stages"][int(shard[3:])])
    raise KeyError(f"unknown shard {shard!r}; have {list(index)}")


def load_fni8_checkpoint(path: str, *, device: str = "cuda", names: list[str] | None = None,
                         shard: str | None = None) -> dict[str, QTensor]:
    """{name: QTensor} on `device` for all tensors, `names`, or one `shard`."""
    with FQReader(path) as r:
        if shard is not None:
            names = _shard_names(r.shards, shard)
        return r.load_many(r.names if names is None else names, device)


def load_fni8_state_dict(path: str, *, device: str = "cuda", names: list[str] | None = None,
                         shard: str | None = None) -> dict:
    """Quantized weights stay QTensor; "raw" entries (norms, embeddings, router
    gate) become their plain tensor."""
    loaded = load_fni8_checkpoint(path, device=device, names=names, shard=shard)
    return {n: (qt.data if qt.scheme == "raw" else qt) for n, qt in loaded.items()}


def checkpoint_info(path: str) -> dict:
    with FQReader(path) as r:
        h = r.header
        return {
            "arch": h["arch"], "quant": h["quant"], "version": h["version"],
            "num_tensors": len(r.names),
            "shards": {k: len(v) for k, v in r.shards.items()},
            "meta": h.get("__meta__", {}),
        }
