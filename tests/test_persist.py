"""Prompt-cache files: format checks that need no GPU."""
import pytest
import torch


def test_rejects_foreign_safetensors(tmp_path):
    from safetensors.torch import save_file

    from chronoquant_mlx_amd import load_prompt_cache
    f = str(tmp_path / "other.safetensors")
    save_file({"0.0": torch.zeros(2)}, f, metadata={"format": "something-else"})
    with pytest.raises(ValueError):
        load_prompt_cache(f, device="cpu")


def test_save_rejects_unknown_cache_type(tmp_path):
    from chronoquant_mlx_amd import save_prompt_cache

    class Foreign:
        state = []
        meta_state = ""
    with pytest.raises(TypeError):
        save_prompt_cache(str(tmp_path / "x.safetensors"), [Foreign()])
