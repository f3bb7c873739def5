"""Checkpoint stacking and the tiny Qwen3-MoE model against the reference's own fixture.

The fixture (``tests/golden/qwen3_moe``: config, checkpoint and ``reference.safetensors``) is the
reference's ``crates/models/tests/it/qwen3/data/qwen3_moe``, whose vectors the reference made with
transformers' ``Qwen3MoeForCausalLM`` in FP32 (crates/models/tests/it/qwen3/reference.rs:1-28).
The model here is a float64 numpy restatement of that architecture whose MoE blocks take their
experts from ``uniserve_moe.checkpoint.stack_experts`` and their routing from the oracle's
``topk_softmax`` (FP32 scores, renormalised): the final hidden states and logits of both rows must
agree within the reference's own bound, ``2 u terms`` relative to the largest magnitude
(reference.rs:14-27, 66-69, 75-131). A wrong stacking order (gate before up), a wrong expert, a
lost renormalisation or a wrong routing changes the rows by far more than that bound.

The fixture's widths (hidden 16, intermediate 8) are below the HIP kernels' 64-element steps, as
they are below the reference's CUDA kernels' (their manifests refuse them too); zero-padded to 64
the blocks are unchanged (checked here on the oracle), and ``test_gpu_checkpoint.py`` runs them so
on the device.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch
from safetensors.torch import load_file

from uniserve_moe.checkpoint import (ExpertNames, quantize_blocks_e4m3, quantize_blocks_mxfp4, router_weight, slot_map,
                                    stack_experts)

FIXTURE = Path(__file__).resolve().parent / "golden" / "qwen3_moe"
UNIT_ROUNDOFF = np.float32(np.finfo(np.float32).eps / 2)


@pytest.fixture(scope="module")
def fixture():
    config = json.loads((FIXTURE / "config.json").read_text())
    tensors = load_file(FIXTURE / "model.safetensors")
    reference = load_file(FIXTURE / "reference.safetensors")
    return config, tensors, reference


def test_modules_layout_stacks_up_before_gate(fixture):
    config, tensors, _ = fixture
    E = config["num_experts"]
    up_gate, down = stack_experts(tensors, "model.layers.1", E)
    I, H = config["moe_intermediate_size"], config["hidden_size"]
    assert tuple(up_gate.shape) == (E, 2 * I, H) and tuple(down.shape) == (E, H, I)
    for e in range(E):
        prefix = f"model.layers.1.mlp.experts.{e}"
        assert torch.equal(up_gate[e, :I], tensors[f"{prefix}.up_proj.weight"])
        assert torch.equal(up_gate[e, I:], tensors[f"{prefix}.gate_proj.weight"])
        assert torch.equal(down[e], tensors[f"{prefix}.down_proj.weight"])
    assert torch.equal(router_weight(tensors, "model.layers.1"), tensors["model.layers.1.mlp.gate.weight"])


def test_stacked_layout_swaps_each_experts_halves(fixture):
    """transformers' fused experts keep gate rows first; the stacks come out up-first all the same."""
    config, tensors, _ = fixture
    E = config["num_experts"]
    fused = dict(tensors)
    fused["model.layers.0.mlp.experts.gate_up_proj"] = torch.stack(
        [torch.cat([tensors[f"model.layers.0.mlp.experts.{e}.gate_proj.weight"],
                    tensors[f"model.layers.0.mlp.experts.{e}.up_proj.weight"]]) for e in range(E)])
    fused["model.layers.0.mlp.experts.down_proj"] = torch.stack(
        [tensors[f"model.layers.0.mlp.experts.{e}.down_proj.weight"] for e in range(E)])
    want = stack_experts(tensors, "model.layers.0", E)
    got = stack_experts(fused, "model.layers.0", E, names=ExpertNames(layout="stacked"))
    assert torch.equal(got[0], want[0]) and torch.equal(got[1], want[1])


def test_order_window_and_split(fixture):
    """Slots follow the order, a window takes contiguous slots, a split takes a rank's rows of up
    and gate and the same columns of down (crates/nn/src/modules/moe.rs:363-378)."""
    config, tensors, _ = fixture
    E, I = config["num_experts"], config["moe_intermediate_size"]
    order = [2, 0, 3, 1]
    whole_up_gate, whole_down = stack_experts(tensors, "model.layers.0", E)
    up_gate, down = stack_experts(tensors, "model.layers.0", E, order=order, window=range(1, 3), split=(1, 2))
    assert tuple(up_gate.shape) == (2, I, config["hidden_size"])
    for index, slot in enumerate(range(1, 3)):
        e = order[slot]
        rows = slice(I // 2, I)
        assert torch.equal(up_gate[index, : I // 2], whole_up_gate[e, :I][rows])
        assert torch.equal(up_gate[index, I // 2:], whole_up_gate[e, I:][rows])
        assert torch.equal(down[index], whole_down[e][:, rows])
    assert slot_map(order).tolist() == [1, 3, 0, 2]
    with pytest.raises(ValueError):
        slot_map([0, 0, 1, 2])
    with pytest.raises(ValueError):
        stack_experts(tensors, "model.layers.0", E, split=(0, 3))


def test_block_quantiser_matches_the_oracle(oracle):
    """The host-side 128 x 128 block quantiser writes the oracle's codes and scales bit for bit."""
    rng = np.random.default_rng(7)
    w = torch.from_numpy(rng.normal(0.0, 0.02, (2, 256, 384)).astype(np.float32)).to(torch.bfloat16)
    w[0, :128, :128] = 0.0                                   # an all-zero block: scale 1
    w[1, 5, 7] = 3.0e4                                       # a block with a large outlier
    codes, scales = quantize_blocks_e4m3(w)
    want_codes, want_scales = oracle.quantize_blocks_fp8(w.view(torch.int16).numpy().view(np.uint16))
    np.testing.assert_array_equal(codes.numpy(), want_codes)
    np.testing.assert_array_equal(scales.numpy().view(np.uint32), want_scales.view(np.uint32))


def test_mxfp4_quantiser_matches_the_oracle(oracle):
    """The host-side MXFP4 quantiser writes the oracle's pairs and E8M0 bytes bit for bit, over
    every rounding tie, signed zeros, an all-zero block, an outlier and blocks whose exponent
    clamps at -127."""
    rng = np.random.default_rng(8)
    w = torch.from_numpy(rng.normal(0.0, 0.02, (3, 64, 256)).astype(np.float32)).to(torch.bfloat16)
    w[0, 0, :32] = 0.0
    ties = [6.0, 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, -0.25, -0.1, -5.0, 4.5, 0.5, 2.75]
    w[0, 1, 32:32 + len(ties)] = torch.tensor(ties)
    w[1, 2, 64:96] = 0.0
    w[1, 2, 70] = -1.0e-38                                   # subnormal amax: exponent clamps at -127
    w[2, 3, 5] = 3.0e4
    pairs, scales = quantize_blocks_mxfp4(w)
    want_pairs, want_scales = oracle.quantize_blocks_mxfp4(w.view(torch.int16).numpy().view(np.uint16))
    np.testing.assert_array_equal(scales.numpy(), want_scales)
    np.testing.assert_array_equal(pairs.numpy(), want_pairs)
    assert scales[0, 0, 0] == 127 and scales[0, 1, 1] == 127


# ---- the tiny model ----------------------------------------------------------------------------


def rms_norm(x, weight, eps):
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * weight


def rope(x, positions, theta):
    """Rotary embedding of ``[T, heads, head_dim]`` (halves rotated, transformers' convention)."""
    half = x.shape[-1] // 2
    inv_freq = 1.0 / theta ** (np.arange(0, 2 * half, 2, dtype=np.float64) / (2 * half))
    angles = positions[:, None] * inv_freq[None, :]
    cos = np.concatenate([np.cos(angles)] * 2, axis=-1)[:, None, :]
    sin = np.concatenate([np.sin(angles)] * 2, axis=-1)[:, None, :]
    rotated = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    return x * cos + rotated * sin


def attention(h, w, config):
    T = h.shape[0]
    heads, kv_heads, dim = config["num_attention_heads"], config["num_key_value_heads"], config["head_dim"]
    eps, theta = config["rms_norm_eps"], config["rope_parameters"]["rope_theta"]
    q = (h @ w("self_attn.q_proj").T).reshape(T, heads, dim)
    k = (h @ w("self_attn.k_proj").T).reshape(T, kv_heads, dim)
    v = (h @ w("self_attn.v_proj").T).reshape(T, kv_heads, dim)
    q = rms_norm(q, w("self_attn.q_norm"), eps)
    k = rms_norm(k, w("self_attn.k_norm"), eps)
    positions = np.arange(T, dtype=np.float64)
    q, k = rope(q, positions, theta), rope(k, positions, theta)
    out = np.empty((T, heads, dim))
    causal = np.triu(np.ones((T, T), dtype=bool), 1)
    for head in range(heads):
        kv = head // (heads // kv_heads)
        scores = q[:, head] @ k[:, kv].T / np.sqrt(dim)
        scores[causal] = -np.inf
        scores = np.exp(scores - scores.max(axis=-1, keepdims=True))
        out[:, head] = (scores / scores.sum(axis=-1, keepdims=True)) @ v[:, kv]
    return out.reshape(T, heads * dim) @ w("self_attn.o_proj").T


def moe_block(h, tensors, prefix, config, oracle):
    """Routing by the oracle (FP32 scores, renormalised), experts from the checkpoint stacks."""
    E, top, I = config["num_experts"], config["num_experts_per_tok"], config["moe_intermediate_size"]
    up_gate, down = (t.double().numpy() for t in stack_experts(dict(tensors), prefix, E))
    router = router_weight(tensors, prefix).double().numpy()
    scores = (h @ router.T).astype(np.float32)
    ids, weights = oracle.topk_softmax(scores, top, renormalize=config["norm_topk_prob"])
    out = np.zeros_like(h)
    for t in range(h.shape[0]):
        for k in range(top):
            e = ids[t, k]
            product = up_gate[e] @ h[t]
            gated = product[I:] / (1.0 + np.exp(-product[I:])) * product[:I]   # silu(gate) * up
            out[t] += float(weights[t, k]) * (down[e] @ gated)
    return out


def forward(ids, tensors, config, oracle):
    w_all = {name: t.double().numpy() for name, t in tensors.items()}
    eps = config["rms_norm_eps"]
    x = w_all["model.embed_tokens.weight"][ids]
    for layer in range(config["num_hidden_layers"]):
        prefix = f"model.layers.{layer}"
        w = lambda name, p=prefix: w_all[f"{p}.{name}.weight"] if f"{p}.{name}.weight" in w_all else w_all[f"{p}.{name}"]  # noqa: E731
        x = x + attention(rms_norm(x, w("input_layernorm"), eps), w, config)
        x = x + moe_block(rms_norm(x, w("post_attention_layernorm"), eps), tensors, prefix, config, oracle)
    hidden = rms_norm(x, w_all["model.norm.weight"], eps)
    return hidden, hidden @ w_all["lm_head.weight"].T


# ---- the blocks at the kernels' widths ------------------------------------------------------------

PAD = 64


def block_inputs(ids, tensors, config, oracle):
    """Each MoE block's input rows in the float64 forward of the fixture's model."""
    w_all = {name: t.double().numpy() for name, t in tensors.items()}
    eps = config["rms_norm_eps"]
    x = w_all["model.embed_tokens.weight"][ids]
    for layer in range(config["num_hidden_layers"]):
        prefix = f"model.layers.{layer}"
        w = lambda name, p=prefix: w_all[f"{p}.{name}.weight"] if f"{p}.{name}.weight" in w_all else w_all[f"{p}.{name}"]  # noqa: E731
        x = x + attention(rms_norm(x, w("input_layernorm"), eps), w, config)
        h = rms_norm(x, w("post_attention_layernorm"), eps)
        yield layer, prefix, h
        x = x + moe_block(h, tensors, prefix, config, oracle)


def padded(up_gate, down, router, H, I):
    """Zero-padded copies at hidden and intermediate PAD: up rows 0..I-1, gate rows PAD..PAD+I-1."""
    E = up_gate.shape[0]
    ug = torch.zeros((E, 2 * PAD, PAD), dtype=torch.float32)
    ug[:, :I, :H] = up_gate[:, :I]
    ug[:, PAD:PAD + I, :H] = up_gate[:, I:]
    dn = torch.zeros((E, PAD, PAD), dtype=torch.float32)
    dn[:, :H, :I] = down
    rt = torch.zeros((E, PAD), dtype=torch.float32)
    rt[:, :H] = router
    return ug, dn, rt


def test_zero_padded_blocks_are_the_checkpoint_s_blocks(fixture, oracle):
    """The oracle's bf16 layer on the zero-padded stacks (hidden and intermediate 64, the HIP
    layer's smallest) against each block of the float64 forward: padding adds nothing, so the
    padded columns come out exactly zero and the rest within the bf16 bar (relative to the peak)."""
    config, tensors, reference = fixture
    E, top = config["num_experts"], config["num_experts_per_tok"]
    H, I = config["hidden_size"], config["moe_intermediate_size"]
    ids = reference["rows.0.ids"].numpy().astype(np.int64)
    for layer, prefix, h in block_inputs(ids, tensors, config, oracle):
        up_gate, down = (t.float() for t in stack_experts(dict(tensors), prefix, E))
        ug, dn, rt = padded(up_gate, down, router_weight(tensors, prefix).float(), H, I)
        x = np.zeros((h.shape[0], PAD), np.float32)
        x[:, :H] = h
        b = lambda a: oracle.bf16_encode(np.asarray(a, np.float32))  # noqa: E731
        out, _, _, _ = oracle.moe_layer(b(x), b(rt.numpy()), b(ug.numpy()), b(dn.numpy()), top)
        got = oracle.bf16_decode(out).astype(np.float64)
        assert (got[:, H:] == 0).all()
        want = moe_block(h, tensors, prefix, config, oracle)
        peak = np.abs(want).max()
        assert np.abs(got[:, :H] - want).max() <= 2e-2 * peak
        assert np.abs(got[:, :H] - want).mean() <= 1e-3 * max(1.0, peak)


def stack_terms(config, keys):
    """The reference's count of reduction terms on the path to an output (reference.rs:75-131),
    for the attention and MoE layers of this fixture."""
    hidden, dim, heads = config["hidden_size"], config["head_dim"], config["num_attention_heads"]
    mixer = hidden + dim + 2 + dim + 2 * keys + 1 + heads * dim
    routed = (hidden + config["num_experts"] + config["num_experts_per_tok"] + hidden + 1
              + config["moe_intermediate_size"] + config["num_experts_per_tok"])
    layer = 2 * hidden + 2 + mixer + routed
    return config["num_hidden_layers"] * layer + hidden


@pytest.mark.parametrize("row", [0, 1])
def test_tiny_qwen3_moe_matches_the_reference(fixture, oracle, row):
    config, tensors, reference = fixture
    ids = reference[f"rows.{row}.ids"].numpy().astype(np.int64)
    hidden, logits = forward(ids, tensors, config, oracle)
    bound = float(2 * UNIT_ROUNDOFF * stack_terms(config, len(ids)))
    for name, got in (("hidden", hidden), ("logits", logits)):
        want = reference[f"rows.{row}.{name}"].double().numpy()
        scale = np.abs(want).max()
        err = np.abs(got - want).max() / scale
        assert err <= bound, f"row {row} {name}: {err:.3g} of the largest magnitude, bound {bound:.3g}"


def test_tiny_model_detects_a_swapped_stack(fixture, oracle):
    """The bound is tight enough to see the stacking order: gate-before-up stacks miss it."""
    config, tensors, reference = fixture
    swapped = dict(tensors)
    for layer in range(config["num_hidden_layers"]):
        for e in range(config["num_experts"]):
            p = f"model.layers.{layer}.mlp.experts.{e}"
            swapped[f"{p}.up_proj.weight"], swapped[f"{p}.gate_proj.weight"] = (
                tensors[f"{p}.gate_proj.weight"], tensors[f"{p}.up_proj.weight"])
    ids = reference["rows.1.ids"].numpy().astype(np.int64)
    _, logits = forward(ids, swapped, config, oracle)
    want = reference["rows.1.logits"].double().numpy()
    bound = float(2 * UNIT_ROUNDOFF * stack_terms(config, len(ids)))
    assert np.abs(logits - want).max() / np.abs(want).max() > 100 * bound
