"""Checkpoints of the reference's training script, loaded into the models of this package.

Layout (scripts/train_imagenet256.py:79-94 writes it with ``torch.save``)::

    {"model": state_dict, "optimizer": optimizer.state_dict(),
     "ema": {parameter name: tensor},             # parameters only, no buffers
     "step": int, "args": dict, "meta": {"model", "prediction", "num_classes", "image_size", "patch_size"}}

Old research checkpoints name the read and write the other way round
(``shared_write`` / ``blocks.*.read``, ``write_logits`` / ``read_weight``);
``migrate_checkpoint_state`` maps them to the current names
(flowmatching_lthc/checkpoint.py:12-14, local_thc.py:41-61).

Files are read with ``torch.load(weights_only=True)``: nothing in a
checkpoint is executed.
"""

from __future__ import annotations

import os
from collections.abc import Iterable, Mapping

import torch

from .model import migrate_lthc_state_dict_keys

CHECKPOINT_KEYS = ("model", "optimizer", "ema", "step", "args", "meta")


def migrate_checkpoint_state(state: Mapping[str, torch.Tensor], keep: set[str] | None = None) -> dict[str, torch.Tensor]:
    """State dict with the current read / write key names (flowmatching_lthc/checkpoint.py:12-14).

    Keys in ``keep`` (the target model's own names) are left as they are.  The migration renames every
    ``.read_weight`` to ``.write_weight``, which is right for the old shared-read checkpoints but would fold a
    v2 model's ``pool.read_weight`` onto its ``pool.write_weight``; the reference's loader does that (a v2
    checkpoint then fails to load strictly, and its EMA read weights are silently not loaded)."""
    state = dict(state)
    if not keep:
        return migrate_lthc_state_dict_keys(state)
    out = migrate_lthc_state_dict_keys({k: v for k, v in state.items() if k not in keep})
    out.update({k: v for k, v in state.items() if k in keep})
    return out


def load_checkpoint(path: str | os.PathLike, map_location: str | torch.device = "cpu") -> dict:
    """Read a checkpoint file with the weights-only loader (tensors, containers and plain values only)."""
    ckpt = torch.load(path, map_location=map_location, weights_only=True)
    if not isinstance(ckpt, Mapping):
        raise ValueError(f"{path}: expected a checkpoint dict, got {type(ckpt).__name__}")
    return dict(ckpt)


def load_model_state(model: torch.nn.Module, ckpt: Mapping, key: str = "ema") -> list[str]:
    """Load the ``model`` or ``ema`` weights of ``ckpt`` into ``model`` (flowmatching_lthc/checkpoint.py:17-41).

    ``key="model"`` loads the full state dict strictly.  ``key="ema"`` takes every entry the EMA holds (the
    EMA stores parameters only) and keeps the model's own values for the rest, such as buffers; the names
    kept are returned.  Old key names are migrated first (names the model itself has are kept as they are).
    Raises ``ValueError`` for another key and ``KeyError`` when the checkpoint has no EMA weights.
    """
    own = set(model.state_dict())
    if key == "model":
        model.load_state_dict(migrate_checkpoint_state(ckpt["model"], own))
        return []
    if key != "ema":
        raise ValueError(f"unsupported checkpoint state key: {key}")
    if "ema" not in ckpt:
        raise KeyError("checkpoint does not contain EMA weights")
    ema = migrate_checkpoint_state(ckpt["ema"], own)
    state = model.state_dict()
    kept = []
    for name in state:
        if name in ema:
            state[name] = ema[name]
        else:
            kept.append(name)
    model.load_state_dict(state)
    return kept


def checkpoint_state(
    model: torch.nn.Module,
    optimizer: torch.optim.Optimizer | None,
    ema_params: Iterable[torch.Tensor] | None,
    step: int,
    args: Mapping | None = None,
    meta: Mapping | None = None,
) -> dict:
    """The reference's checkpoint dict (scripts/train_imagenet256.py:79-94).

    ``ema_params`` follow ``model.named_parameters()`` order, as the reference's EMA list does; ``meta``
    defaults to the fields the reference fills from ``args`` and the model.
    """
    args = dict(args or {})
    names = [n for n, _ in model.named_parameters()]
    ema = None
    if ema_params is not None:
        ema_params = list(ema_params)
        if len(ema_params) != len(names):
            raise ValueError(f"{len(ema_params)} EMA tensors for {len(names)} parameters")
        ema = {n: e.detach().cpu() for n, e in zip(names, ema_params)}
    if meta is None:
        meta = {
            "model": args.get("model"),
            "prediction": args.get("prediction"),
            "num_classes": 1000,
            "image_size": getattr(model, "input_size", 256),
            "patch_size": getattr(model, "patch_size", 16),
        }
    return {
        "model": model.state_dict(),
        "optimizer": optimizer.state_dict() if optimizer is not None else None,
        "ema": ema,
        "step": int(step),
        "args": args,
        "meta": dict(meta),
    }


def save_checkpoint(path: str | os.PathLike, *a, **kw) -> None:
    """``torch.save`` of ``checkpoint_state(*a, **kw)``; the file loads with ``load_checkpoint``."""
    torch.save(checkpoint_state(*a, **kw), path)
