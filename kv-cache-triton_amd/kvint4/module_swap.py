"""In-place replacement of a model's attention modules, shared by every family.

The reference has one swap routine per family (``models/llama3/llama3_quant.py:146-204``
rebinds the four projection Parameters and moves accelerate hooks;
``models/gpt2/gpt2_quant.py:141-157`` copies a state dict into a fresh module).
Both public entry points here keep their contracts (same names, a ``ValueError``
when the model has no decoder blocks, a repeated call only updates the group
size) and share this routine:

* The replacement module is constructed on the ``meta`` device, so building it
  allocates no weights.
* Every Parameter and buffer of the old module is rebound into the new one
  under the same name (the new module then owns the very tensors the old one
  had: same device, dtype and storage; nothing is copied). A name the new
  module has and the old one lacks raises, so no meta tensor survives.
* An accelerate hook found on the old module or on any of its submodules is
  detached there first (which puts offloaded weights back on the module), and
  attached to the module of the same name in the new one after the rebinding.
  A hook that cannot be moved raises ``RuntimeError``; nothing is skipped
  silently (an offloaded projection without its hook would run on the wrong
  device or with its weights still offloaded).
"""

from __future__ import annotations

from typing import Callable, Sequence

import torch


def _hook_tools():
    try:
        from accelerate.hooks import add_hook_to_module, remove_hook_from_module
    except ImportError as exc:  # a hooked model without accelerate cannot be swapped safely
        raise RuntimeError("the model carries accelerate hooks but accelerate cannot be imported") from exc
    return add_hook_to_module, remove_hook_from_module


def _rebind_tensors(old: torch.nn.Module, new: torch.nn.Module) -> None:
    """Give ``new`` the Parameters and buffers of ``old``, name by name."""
    old_mods = dict(old.named_modules())
    for mod_name, dst in new.named_modules():
        src = old_mods.get(mod_name)
        for pname, _ in list(dst.named_parameters(recurse=False)):
            if src is None or pname not in src._parameters:
                raise RuntimeError(f"attention swap: the replacement has parameter "
                                   f"'{mod_name + '.' if mod_name else ''}{pname}' that the original lacks")
        for bname, _ in list(dst.named_buffers(recurse=False)):
            if src is None or bname not in src._buffers:
                raise RuntimeError(f"attention swap: the replacement has buffer "
                                   f"'{mod_name + '.' if mod_name else ''}{bname}' that the original lacks")
        if src is None:
            continue
        for pname, p in src._parameters.items():
            if pname in dst._parameters or p is None:
                dst._parameters[pname] = p
        for bname, b in src._buffers.items():
            if bname in dst._buffers:
                dst._buffers[bname] = b


def _detach_hooks(old: torch.nn.Module, new: torch.nn.Module) -> list:
    """Detach every accelerate hook of ``old`` (which restores any offloaded
    weights onto the module) and return (target submodule of ``new``, hook)."""
    hooked = [(name, mod) for name, mod in old.named_modules() if getattr(mod, "_hf_hook", None) is not None]
    if not hooked:
        return []
    _, remove_hook = _hook_tools()
    new_mods = dict(new.named_modules())
    moves = []
    for name, src in hooked:
        dst = new_mods.get(name)
        if dst is None:
            raise RuntimeError(f"attention swap: no submodule '{name}' in the replacement to take its accelerate hook")
        moves.append((dst, src._hf_hook))
    for _, src in hooked:
        remove_hook(src)
    return moves


def _attach_hooks(moves: list) -> None:
    if moves:
        add_hook, _ = _hook_tools()
        for dst, hook in moves:
            add_hook(dst, hook)


def swap_attention_modules(blocks: Sequence[torch.nn.Module], attr: str, quant_cls: type,
                           build: Callable[[torch.nn.Module], torch.nn.Module], group_size: int) -> int:
    """Replace ``block.<attr>`` of every block by ``build(old)`` (constructed on
    the meta device, then given the old module's tensors and hooks). Blocks
    whose module already is a ``quant_cls`` only get ``quant_group_size``
    updated. Returns the number of modules replaced."""
    replaced = 0
    for block in blocks:
        old = getattr(block, attr)
        if isinstance(old, quant_cls):
            old.quant_group_size = int(group_size)
            continue
        with torch.device("meta"):
            new = build(old)
        moves = _detach_hooks(old, new)
        _rebind_tensors(old, new)
        _attach_hooks(moves)
        new.train(old.training)
        setattr(block, attr, new)
        replaced += 1
    return replaced
