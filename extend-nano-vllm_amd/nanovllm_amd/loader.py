"""safetensors checkpoint loading from a local directory
(nanovllm/utils/loader.py:12-67).

Fused parameters (QKV, gate_up) are filled shard by shard through the
parameter's ``weight_loader``; a model may claim tensors first with a
``load_weight(name, tensor) -> bool`` hook; a tied LM head accepts
``model.embed_tokens.weight``.
"""
import os
from glob import glob

import torch
from safetensors import safe_open
from torch import nn


def _default_loader(param: nn.Parameter, loaded: torch.Tensor) -> None:
    param.data.copy_(loaded)


def checkpoint_files(path: str) -> list[str]:
    return sorted(glob(os.path.join(path, "*.safetensors")))


def load_model(model: nn.Module, path: str) -> int:
    """Load every tensor of the directory's *.safetensors files into ``model``;
    returns the number of tensors consumed."""
    packed = getattr(model, "packed_modules_mapping", {})
    hook = getattr(model, "load_weight", None)
    params = dict(model.named_parameters())
    used = 0
    files = checkpoint_files(path)
    if not files:
        raise FileNotFoundError(f"no *.safetensors files in {path} (use load_format='dummy' "
                                "for random weights)")
    for file in files:
        with safe_open(file, "pt", "cpu") as f:
            for name in f.keys():
                tensor = f.get_tensor(name)
                if hook is not None and hook(name, tensor):
                    used += 1
                    continue
                target = None
                shard = None
                for key, (fused, shard_id) in packed.items():
                    if key in name:
                        target = params.get(name.replace(key, fused))
                        shard = shard_id
                        break
                if shard is not None:
                    if target is not None:
                        target.weight_loader(target, tensor, shard)
                        used += 1
                    continue
                target = params.get(name)
                if (target is None and name == "model.embed_tokens.weight"
                        and getattr(model, "tie_word_embeddings", False)):
                    target = params.get("lm_head.weight")
                if target is None:
                    continue
                getattr(target, "weight_loader", _default_loader)(target, tensor)
                used += 1
    return used
