"""Expert stacks from a checkpoint's tensors, in the arrangement the grouped products read.

The reference loads a block's dense experts as two stacks (crates/nn/src/modules/moe.rs:345-451,
``MoE::load_dense``): ``up_gate`` ``[slots, 2 * intermediate, hidden]`` with each expert's up rows
before its gate rows, and ``down`` ``[slots, hidden, intermediate]``. A checkpoint stores them in
one of two layouts (``ExpertLayout``, moe.rs:135-149):

* ``modules``: one module per expert, ``<list>.<e>.<up|gate|down>.weight`` (Qwen3-MoE's
  ``mlp.experts.<e>.up_proj.weight`` ...), each ``[intermediate, hidden]`` (``down``
  ``[hidden, intermediate]``);
* ``stacked``: two tensors under the list (transformers' fused experts), ``gate_up``
  ``[experts, 2 * intermediate, hidden]`` with each expert's *gate* rows before its up rows, and
  ``down`` ``[experts, hidden, intermediate]``; loading swaps each expert's halves.

Slots: the stacks are laid out in slot order, ``order[s]`` the expert stored at slot ``s``
(``MoEConfig::order``, moe.rs:112-116); the router's ids become slots through ``slot_map(order)``,
the ``map`` argument of topk_softmax. A rank holds one contiguous window of the slots, and a
tensor-parallel rank ``r`` of ``n`` holds rows ``[r * I / n, (r + 1) * I / n)`` of each up and gate
projection and the same columns of each down projection (moe.rs:363-378).

Everything here is host-side tensor plumbing (torch CPU or device tensors alike); nothing runs a
kernel. It is a loader and test-harness helper beside the product, not part of the drop-in: the
drop-in boundary is the C ABI (include/*.h), which takes the stacks as plain device pointers
however they were built.
"""

from dataclasses import dataclass

import torch

__all__ = [
    "ExpertNames",
    "QWEN3_MOE",
    "stack_experts",
    "router_weight",
    "slot_map",
    "quantize_blocks_e4m3",
]


@dataclass(frozen=True)
class ExpertNames:
    """Where a block's experts sit in a checkpoint, relative to the block's prefix."""

    router: str = "mlp.gate"
    list: str = "mlp.experts"
    up: str = "up_proj"
    gate: str = "gate_proj"
    down: str = "down_proj"
    layout: str = "modules"           # or "stacked"
    stacked_gate_up: str = "gate_up_proj"
    stacked_down: str = "down_proj"


QWEN3_MOE = ExpertNames()


def _join(*parts):
    return ".".join(p for p in parts if p)


def router_weight(tensors, prefix, names=QWEN3_MOE):
    """The router's ``[experts, hidden]`` weight."""
    return tensors[_join(prefix, names.router, "weight")]


def slot_map(order):
    """``map[e]`` = the slot expert ``e`` is stored at, for ``order[s]`` = the expert at slot ``s``."""
    order = [int(e) for e in order]
    if sorted(order) != list(range(len(order))):
        raise ValueError("an expert order is a permutation of the experts")
    mapping = [0] * len(order)
    for slot, expert in enumerate(order):
        mapping[expert] = slot
    return torch.tensor(mapping, dtype=torch.int32)


def stack_experts(tensors, prefix, experts, names=QWEN3_MOE, order=None, window=None, split=(0, 1)):
    """The ``(up_gate, down)`` stacks of the slots ``window`` (a range; all slots by default).

    ``tensors`` maps checkpoint names to tensors; ``prefix`` is the block's module path
    (``model.layers.<l>``). ``split`` = ``(rank, size)`` takes a tensor-parallel rank's block of
    every expert's intermediate width.
    """
    order = list(range(experts)) if order is None else [int(e) for e in order]
    if len(order) != experts:
        raise ValueError("the expert order names every expert once")
    slot_map(order)  # validates the permutation
    window = range(experts) if window is None else window
    if len(window) == 0 or window[0] < 0 or window[-1] >= experts:
        raise ValueError("the window lies outside the slots")
    rank, size = split
    if size < 1 or not 0 <= rank < size:
        raise ValueError("a split is (rank, size) with 0 <= rank < size")

    def projections(expert):
        if names.layout == "modules":
            module = lambda name: tensors[_join(prefix, names.list, str(expert), name, "weight")]  # noqa: E731
            return module(names.up), module(names.gate), module(names.down)
        if names.layout == "stacked":
            gate_up = tensors[_join(prefix, names.list, names.stacked_gate_up)][expert]
            down = tensors[_join(prefix, names.list, names.stacked_down)][expert]
            half = gate_up.shape[0] // 2
            return gate_up[half:], gate_up[:half], down
        raise ValueError(f"unknown expert layout {names.layout!r}")

    up_gates, downs = [], []
    for slot in window:
        up, gate, down = projections(order[slot])
        intermediate, hidden = up.shape
        if gate.shape != up.shape or tuple(down.shape) != (hidden, intermediate):
            raise ValueError(f"expert {order[slot]}'s projections disagree on their extents")
        if intermediate % size != 0:
            raise ValueError("the split does not divide the intermediate width")
        local = intermediate // size
        rows = slice(rank * local, (rank + 1) * local)
        up_gates.append(torch.cat([up[rows], gate[rows]], dim=0))
        downs.append(down[:, rows])
    return torch.stack(up_gates).contiguous(), torch.stack(downs).contiguous()


def quantize_blocks_e4m3(stack, block=128):
    """OCP e4m3fn codes of a ``[stacks, N, K]`` stack with one FP32 scale per ``block x block``
    block: scale = blockmax / 448 (1 for an all-zero block), codes = e4m3(w / scale), nearest-even
    and saturating. Returns ``(codes uint8 [stacks, N, K], scales f32 [stacks, N/block, K/block])``.
    """
    stacks, n, k = stack.shape
    if n % block or k % block:
        raise ValueError("the stack's extents are not whole blocks")
    blocks = stack.float().reshape(stacks, n // block, block, k // block, block)
    amax = blocks.abs().amax(dim=(2, 4), keepdim=True)
    scale = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
    codes = (blocks / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return (codes.reshape(stacks, n, k).view(torch.uint8).contiguous(),
            scale.reshape(stacks, n // block, k // block).contiguous())


def quantize_blocks_mxfp4(stack):
    """OCP MXFP4 form of a ``[stacks, N, K]`` stack: one E8M0 scale byte per 32 consecutive K
    elements, the smallest power of two 2^e with ``blockmax <= 6 * 2^e`` (2^0 for an all-zero
    block, e clamped to [-127, 127]), and E2M1 codes of ``w / 2^e`` rounded to nearest, ties to
    the even code, saturating at 6; two codes per byte, the lower K index in the low nibble.
    Returns ``(pairs uint8 [stacks, N, K/2], scales uint8 [stacks, N, K/32])``.
    """
    stacks, n, k = stack.shape
    if k % 32:
        raise ValueError("the stack's K extent is not whole 32-element blocks")
    blocks = stack.float().reshape(stacks, n, k // 32, 32)
    amax = blocks.abs().amax(dim=3, keepdim=True)
    live = (amax > 0) & torch.isfinite(amax)
    safe = torch.where(live, amax, torch.ones_like(amax))
    e = torch.frexp(safe / 6.0).exponent.to(torch.int32)
    # amax / 6 rounds; settle the exponent on exact power-of-two comparisons.
    e = torch.where(safe <= torch.ldexp(torch.full_like(safe, 6.0), (e - 1).float()), e - 1, e)
    e = torch.where(safe > torch.ldexp(torch.full_like(safe, 6.0), e.float()), e + 1, e)
    e = torch.where(live, e.clamp(-127, 127), torch.zeros_like(e))
    scaled = blocks / torch.ldexp(torch.ones_like(safe), e.float())
    a = scaled.abs()
    # Midpoints between neighbouring magnitudes 0, .5, 1, 1.5, 2, 3, 4, 6; a tie takes the even code.
    code = ((a > 0.25).int() + (a >= 0.75).int() + (a > 1.25).int() + (a >= 1.75).int() + (a > 2.5).int() +
            (a >= 3.5).int() + (a > 5.0).int())
    code = torch.where(torch.isnan(scaled), torch.zeros_like(code), code | (torch.signbit(scaled).int() << 3))
    code = code.to(torch.uint8).reshape(stacks, n, k // 2, 2)
    pairs = code[..., 0] | (code[..., 1] << 4)
    return pairs.contiguous(), (e + 127).to(torch.uint8).reshape(stacks, n, k // 32).contiguous()
