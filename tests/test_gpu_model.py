"""The backend inside a transformers Qwen2 model (the plugin boundary,
attention.py:57): a full prefill and the split-last-token flow of
evaluate.py:357-380 (prefill S - 1 tokens, then one cached decode step) give the
same last-position logits, for dense and for a V1-routed sparse method."""

import pytest
import torch

from exp3_amd import attention

pytestmark = pytest.mark.gpu

LENGTH = 700   # S - 1 = 699: the split prefill ends inside a partial block


@pytest.fixture()
def small_model(gpu):
    transformers = pytest.importorskip("transformers")
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    saved = ALL_ATTENTION_FUNCTIONS["sdpa"]
    backend = attention.AttentionBackend(alpha=0.08)     # registers as "sdpa"
    cfg = transformers.Qwen2Config(
        vocab_size=1000, hidden_size=3584, intermediate_size=512, num_hidden_layers=2,
        num_attention_heads=28, num_key_value_heads=4, rms_norm_eps=1e-6, rope_theta=1e6,
        max_position_embeddings=4096, tie_word_embeddings=False, use_sliding_window=False,
        attn_implementation="sdpa", torch_dtype="bfloat16")
    torch.manual_seed(5)
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device("cuda"):
            model = transformers.Qwen2ForCausalLM(cfg)
    finally:
        torch.set_default_dtype(torch.float32)
    model.eval()
    try:
        yield model, backend
    finally:
        ALL_ATTENTION_FUNCTIONS["sdpa"] = saved


@pytest.mark.parametrize("method", ("dense", "mean_native"))
def test_split_last_token_matches_full_prefill(small_model, method):
    model, backend = small_model
    backend.configure(method, 0.08)
    ids = torch.randint(0, 1000, (1, LENGTH), generator=torch.Generator().manual_seed(9)).cuda()
    with torch.no_grad():
        full = model(ids, use_cache=True, logits_to_keep=1).logits[:, -1].float()
        pre = model.model(input_ids=ids[:, :-1], use_cache=True)
        step = model(input_ids=ids[:, -1:], past_key_values=pre.past_key_values, use_cache=True,
                     cache_position=torch.tensor([LENGTH - 1], device="cuda"),
                     logits_to_keep=1).logits[:, -1].float()
    assert torch.isfinite(full).all() and torch.isfinite(step).all()
    # same attention over the same keys, bf16 activations through two layers:
    # max |diff| within 2 % of the logit range, and the same greedy token unless
    # the top two logits are closer than that difference
    span = (full.max() - full.min()).item()
    diff = (full - step).abs().max().item()
    assert diff <= 0.02 * span
    top2 = full[0].topk(2).values
    if (top2[0] - top2[1]).item() > 2 * diff:
        assert int(full.argmax()) == int(step.argmax())
