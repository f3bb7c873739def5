"""The HIP layer on experts stacked from the reference's tiny Qwen3-MoE checkpoint.

The fixture (``tests/golden/qwen3_moe``, the reference's crates/models/tests/it/qwen3/data/qwen3_moe)
has MoE blocks of hidden 16, intermediate 8, 4 experts, top 2: below the kernels' 64-element steps
(and the reference's CUDA kernels', whose manifests refuse them too). Zero padding keeps every
product exact: hidden columns 16..63 of x and of the router, and rows / columns of both stacks past
the checkpoint's, contribute nothing to any sum, and a zero up row gates to zero whatever its gate.
So each block runs on the HIP layer at hidden 64 and intermediate 64, its up and gate halves each
padded separately (up rows 0..7 of 0..63, gate rows 64..71), with the stacks built by
``uniserve_moe.checkpoint.stack_experts`` from the checkpoint names.

Inputs are the blocks' own activations: the float64 forward of the fixture's rows (whose hidden
states and logits match the reference's vectors within its bound, ``test_checkpoint.py``) up to
each block's post-attention norm. Against that forward's block output (FP32 routing scores,
float64 experts): the bf16 bar over tokens whose routes agree; a token whose routes differ must
be a near tie of its scores within what rounding to bf16 moves them. Against the oracle's bf16
evaluation of the same padded values: routes bit for bit and BASELINE's full bf16 bar.
"""

import numpy as np
import pytest
import torch

import oracle_lib as oracle
from gpu_helpers import announce, assert_bf16_bar, bf16_values
from test_checkpoint import PAD, block_inputs, fixture, moe_block, padded  # noqa: F401 (fixture)
from uniserve_moe import ops
from uniserve_moe.checkpoint import router_weight, stack_experts

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("row", [0, 1])
def test_moe_blocks_of_the_tiny_checkpoint_on_the_device(device, fixture, row):  # noqa: F811
    config, tensors, reference = fixture
    E, top = config["num_experts"], config["num_experts_per_tok"]
    H, I = config["hidden_size"], config["moe_intermediate_size"]
    token_ids = reference[f"rows.{row}.ids"].numpy().astype(np.int64)
    for layer, prefix, h in block_inputs(token_ids, tensors, config, oracle):
        announce("checkpoint block", row, layer)
        up_gate, down = (t.float() for t in stack_experts(dict(tensors), prefix, E))
        ug, dn, rt = padded(up_gate, down, router_weight(tensors, prefix).float(), H, I)
        T = h.shape[0]
        x = torch.zeros((T, PAD), dtype=torch.float32)
        x[:, :H] = torch.from_numpy(h)
        bf = lambda t: t.to(torch.bfloat16).to(device)  # noqa: E731
        layer_op = ops.MoeLayer(PAD, E, top, PAD, T)
        out = layer_op(bf(x), bf(rt), bf(ug), bf(dn))
        torch.cuda.synchronize()
        got = bf16_values(out)
        assert (got[:, H:] == 0).all(), "padding columns stay zero"
        want = moe_block(h, tensors, prefix, config, oracle)
        router = router_weight(tensors, prefix).double().numpy()
        scores = h @ router.T
        want_ids, _ = oracle.topk_softmax(scores.astype(np.float32), top, renormalize=config["norm_topk_prob"])
        ids = layer_op.view("ids", torch.int32, (T, top)).cpu().numpy()
        agree = (np.sort(ids, axis=1) == np.sort(want_ids, axis=1)).all(axis=1)
        magnitude = np.abs(h) @ np.abs(router).T
        for t in np.flatnonzero(~agree):
            for a, b in zip(sorted(set(want_ids[t]) - set(ids[t])), sorted(set(ids[t]) - set(want_ids[t]))):
                assert abs(scores[t, a] - scores[t, b]) <= 2.0**-7 * (magnitude[t, a] + magnitude[t, b]), (t, a, b)
        assert agree.mean() >= 0.5
        # Against the float64 block the inputs' rounding into bf16 (the checkpoint is FP32) counts
        # too, so only the max-relative bar; against the oracle's bf16 evaluation of the same
        # padded bf16 values, BASELINE's full bar and bit-exact routes.
        assert_bf16_bar(got[agree, :H], want[agree], f"checkpoint row {row} layer {layer}", mean_abs=np.inf)
        b = lambda t: oracle.bf16_encode(t.numpy())  # noqa: E731
        same_bits, same_ids, _, _ = oracle.moe_layer(b(x), b(rt), b(ug), b(dn), top)
        np.testing.assert_array_equal(ids, same_ids)
        assert_bf16_bar(got, oracle.bf16_decode(same_bits), f"checkpoint row {row} layer {layer} (bf16 oracle)")
