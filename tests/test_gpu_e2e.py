"""The Qwen-style decoder (configs[4]'s architecture at a small size) running
on ChronoQuant caches through the patched SDPA symbol."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _tiny():
    from chronoquant_mlx_amd.models.qwen import ModelArgs, random_model
    args = ModelArgs(hidden_size=512, num_hidden_layers=2, num_attention_heads=8,
                     num_key_value_heads=2, head_dim=128, intermediate_size=1024,
                     vocab_size=1000, max_position=4096)
    return random_model(args, seed=1)


@pytest.fixture(autouse=True)
def _patched():
    from chronoquant_mlx_amd import patch
    patch.apply()
    yield
    patch.revert()


def test_graph_decode_equals_eager():
    from chronoquant_mlx_amd import create_full_throttle_caches
    from chronoquant_mlx_amd.models.qwen import generate
    model = _tiny()
    prompt = torch.randint(0, 1000, (1, 700), generator=torch.Generator().manual_seed(2)).cuda()
    c1 = create_full_throttle_caches(model)
    toks_g, _, _ = generate(model, c1, prompt, 40, prefill_chunk=256, graph=True)
    c2 = create_full_throttle_caches(model)
    toks_e, _, _ = generate(model, c2, prompt, 40, prefill_chunk=256, graph=False)
    assert torch.equal(toks_g, toks_e)
    for a, b in zip(c1, c2):
        assert a.offset == b.offset == 700 + 39
        for x, y in zip(a.state, b.state):
            assert torch.equal(x.view(torch.int16) if x.dtype == torch.float16 else x,
                               y.view(torch.int16) if y.dtype == torch.float16 else y)


def test_prefill_kernel_matches_fallback_first_layer():
    # The first layer sees identical K/V in both runs, so its attention output
    # must agree within the attention bar.  Deeper layers are not compared:
    # one-ulp bf16 differences upstream move some residuals across a
    # quantisation boundary, and the two runs then hold different caches.
    from chronoquant_mlx_amd import attention as A
    from chronoquant_mlx_amd import create_full_throttle_caches
    model = _tiny()
    prompt = torch.randint(0, 1000, (1, 300), generator=torch.Generator().manual_seed(3)).cuda()
    outs = []
    h = model.layers[0].self_attn.register_forward_hook(
        lambda m, i, o: outs.append(o.detach().float().clone()))
    try:
        with torch.no_grad():
            model(prompt, create_full_throttle_caches(model))
            A.PREFILL_KERNEL = False
            model(prompt, create_full_throttle_caches(model))
    finally:
        A.PREFILL_KERNEL = True
        h.remove()
    got, ref = outs
    assert ((got - ref).abs() <= 2e-3 + 1e-2 * ref.abs()).all()
    assert ((got - ref).norm() / ref.norm()).item() <= 5e-3


def test_kv_bytes_accounting():
    from chronoquant_mlx_amd import create_full_throttle_caches, synth
    model = _tiny()
    prompt = torch.randint(0, 1000, (1, 500), generator=torch.Generator().manual_seed(4)).cuda()
    caches = create_full_throttle_caches(model)
    with torch.no_grad():
        model(prompt, caches)
    per_layer = synth.compressed_bytes(500, 2, 128, 64, 32)
    assert all(c.nbytes == per_layer for c in caches)
