"""A small ModernBERT Laya checkpoint directory for tests that go through ``Engine``/``Laya`` the way a
user does (laya_cuda/models.py:1-58 file layout): an offline-trained byte-pair tokenizer, configs
with global and local layers and head transformer layers, and seeded safetensors weights."""
import laya_cuda.synthetic as S


def write(root, *, max_len=128, head_max_len=48, layers=4, width=64, heads=1, intermediate=128, head_layers=1,
          seed=3, mfma_dtype="float16"):
    """Writes the checkpoint under ``root``; returns (path, adapter spec, flat weights)."""
    config = S.modernbert_config(layers, width, heads, intermediate, S.tokenizer().get_vocab_size(), 512,
                                 global_every=3, local_attention=64)
    task = {"max_len": max_len, "head_max_len": head_max_len, "head_layers": head_layers,
            "act_costs": {"defer": 0.05}, "temperature": [1.0, 0.7, 1.3],
            "temperature_by_options": {"choice:3-5": 0.8}, "mfma_dtype": mfma_dtype}
    return S.checkpoint(root, config, task, seed=seed)
