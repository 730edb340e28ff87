"""Fuse neighbouring KernelIR ops of the decode step into single kernels.

Runs after lowering, in the ``fast`` numerical mode only.  Every rewrite
replaces a short chain of ``kernel.hip.*`` ops with one ``kernel.hip.*`` op
whose kernel produces bit-identical results (the fused kernels reuse the
single kernels' arithmetic and only remove launches and round trips through
memory):

  rms_norm -> 1..3 linears on its result            kernel.hip.norm_linear_group
  rms_norm -> gate, up linears -> swiglu            kernel.hip.norm_linear_swiglu
  linear -> add (with a residual)                   kernel.hip.linear_residual
  rope -> kv_store of the rotated key               kernel.hip.rope_kv_store
  rope_kv_store -> kv.advance of the same slot      kernel.hip.rope_kv_store (advance)
  rope_kv_store (advance 1) -> decode_attention     kernel.hip.rope_store_attention

A chain is fused only when its intermediate values have no other user and
are not returned, so no value the program can observe disappears.  The
reference has no such pass; its Triton path runs each of these ops as its
own kernel (backends/triton_executor.py:69-130).
"""

from __future__ import annotations

from collections import Counter, defaultdict

from ..ir import Function, Module, Operation
from ..pass_manager import CompilerPass, PassResult



MAX_GROUP_FEATURES = 16384
# A head at least this wide (1024 blocks of 16 features) runs on the wide
# decode kernel, which takes the norm into its input staging.
WIDE_FEATURES = 16384


class FuseDecodeKernelsPass(CompilerPass):
    name = "fuse-decode-kernels"

    def run(self, module: Module) -> PassResult:
        fused: Counter[str] = Counter()
        for function in module.functions:
            fused.update(_fuse_function(function))
        return PassResult(self.name, bool(fused), {"fused": dict(sorted(fused.items()))})


def _uses(function: Function) -> dict[int, list[tuple[int, int]]]:
    """id(value) -> [(op index, operand index)]; a return counts as a use at
    index len(operations)."""

    uses: dict[int, list[tuple[int, int]]] = defaultdict(list)
    for index, operation in enumerate(function.block.operations):
        for position, operand in enumerate(operation.operands):
            uses[id(operand)].append((index, position))
    end = len(function.block.operations)
    for position, value in enumerate(function.returns):
        uses[id(value)].append((end, position))
    return uses


def _producers(function: Function) -> dict[int, int]:
    return {id(result): index
            for index, operation in enumerate(function.block.operations)
            for result in operation.results}


def _fuse_function(function: Function) -> Counter[str]:
    counts: Counter[str] = Counter()
    # Each rule runs to a fixed point before the next so that the SwiGLU rule
    # sees the gate/up linears before the group rule could claim them.
    for rule in (_fuse_swiglu, _fuse_group, _fuse_residual, _fuse_rope_store, _fuse_store_advance,
                 _fuse_store_attention):
        while True:
            name = rule(function)
            if name is None:
                break
            counts[name] += 1
    return counts


def _replace(function: Function, remove: list[int], insert_at: int, new: Operation) -> None:
    ops = function.block.operations
    keep = [op for i, op in enumerate(ops[:insert_at]) if i not in remove]
    keep.append(new)
    keep += [op for i, op in enumerate(ops[insert_at:], start=insert_at) if i not in remove]
    function.block.operations[:] = keep


def _only_used_by(uses, value, index: int) -> bool:
    return all(user == index for user, _ in uses[id(value)])


def _is_norm(operation: Operation) -> bool:
    # A norm that carries a profile-derived lowering plan is dispatched by
    # that plan, so it is not folded into a linear.
    return (operation.name == "kernel.hip.rms_norm"
            and operation.attributes.get("round_before_weight") is True
            and "output_dtype" not in operation.attributes
            and "lowering_plan" not in operation.attributes)


def _fuse_swiglu(function: Function) -> str | None:
    ops = function.block.operations
    uses, producer = _uses(function), _producers(function)
    for s_index, swiglu in enumerate(ops):
        if swiglu.name != "kernel.hip.swiglu" or len(swiglu.operands) != 2:
            continue
        gate, up = swiglu.operands
        g_index, u_index = producer.get(id(gate)), producer.get(id(up))
        if g_index is None or u_index is None or g_index == u_index:
            continue
        g_op, u_op = ops[g_index], ops[u_index]
        if g_op.name != "kernel.hip.linear" or u_op.name != "kernel.hip.linear":
            continue
        if len(g_op.operands) != 2 or len(u_op.operands) != 2:
            continue  # the MLP projections carry no bias
        if g_op.operands[0] is not u_op.operands[0]:
            continue
        if not (_only_used_by(uses, gate, s_index) and _only_used_by(uses, up, s_index)):
            continue
        x = g_op.operands[0]
        n_index = producer.get(id(x))
        if n_index is None or not _is_norm(ops[n_index]):
            continue
        if sorted(user for user, _ in uses[id(x)]) != sorted({g_index, u_index}):
            continue
        norm = ops[n_index]
        new = Operation(
            "kernel.hip.norm_linear_swiglu",
            [norm.operands[0], norm.operands[1], g_op.operands[1], u_op.operands[1]],
            list(swiglu.results),
            {
                "epsilon": norm.attributes["epsilon"],
                "features": g_op.attributes.get("output_features"),
                "fused_from": ["kernel.hip.rms_norm", "kernel.hip.linear", "kernel.hip.linear",
                               "kernel.hip.swiglu"],
                "lowered_from": "serve.rms_norm+serve.linear+serve.linear+serve.swiglu",
            },
        )
        _replace(function, [n_index, g_index, u_index, s_index], s_index, new)
        return new.name
    return None


def _fuse_group(function: Function) -> str | None:
    ops = function.block.operations
    uses, producer = _uses(function), _producers(function)
    for n_index, norm in enumerate(ops):
        if not _is_norm(norm):
            continue
        x = norm.results[0]
        users = uses[id(x)]
        if not 1 <= len(users) <= 3:
            continue
        # Every workgroup of the fused kernel re-normalises the input rows, so
        # it pays for projections of modest width (Q/K/V) and for a single
        # vocabulary-sized head, whose kernel normalises while its first
        # weight loads are in flight; not for wide groups in between.
        widths = [ops[i].attributes.get("output_features") if i < len(ops) else None
                  for i, _ in users]
        if any(not isinstance(n, int) for n in widths):
            continue
        if sum(widths) > MAX_GROUP_FEATURES and not (len(widths) == 1 and widths[0] >= WIDE_FEATURES):
            continue
        linears = [ops[i] if i < len(ops) else None for i, _ in users]
        if any(op is None or op.name != "kernel.hip.linear" for op in linears):
            continue
        if any(position != 0 for _, position in users):
            continue
        operands = [norm.operands[0], norm.operands[1]]
        # The group op takes the norm's place: weights and biases must already
        # be defined there (they are function arguments in the models).
        if any(producer.get(id(operand), -1) >= n_index
               for op in linears for operand in op.operands[1:]):
            continue
        has_bias = []
        for op in linears:
            operands.append(op.operands[1])
            if len(op.operands) == 3:
                operands.append(op.operands[2])
            has_bias.append(len(op.operands) == 3)
        results = [op.results[0] for op in linears]
        new = Operation(
            "kernel.hip.norm_linear_group",
            operands,
            results,
            {
                "epsilon": norm.attributes["epsilon"],
                "has_bias": has_bias,
                "output_features": [op.attributes.get("output_features") for op in linears],
                "fused_from": ["kernel.hip.rms_norm"] + ["kernel.hip.linear"] * len(linears),
                "lowered_from": "serve.rms_norm+" + "+".join(["serve.linear"] * len(linears)),
            },
        )
        remove = [n_index] + [i for i, _ in users]
        _replace(function, remove, n_index, new)
        return new.name
    return None


def _fuse_residual(function: Function) -> str | None:
    ops = function.block.operations
    uses, producer = _uses(function), _producers(function)
    for a_index, add in enumerate(ops):
        if add.name != "kernel.hip.add" or len(add.operands) != 2:
            continue
        for which in (1, 0):
            y = add.operands[which]
            residual = add.operands[1 - which]
            l_index = producer.get(id(y))
            if l_index is None or ops[l_index].name != "kernel.hip.linear":
                continue
            if not _only_used_by(uses, y, a_index) or len(uses[id(y)]) != 1:
                continue
            if residual is y:
                continue
            linear = ops[l_index]
            has_bias = len(linear.operands) == 3
            new = Operation(
                "kernel.hip.linear_residual",
                list(linear.operands) + [residual],
                list(add.results),
                {
                    "has_bias": has_bias,
                    "output_features": linear.attributes.get("output_features"),
                    "fused_from": ["kernel.hip.linear", "kernel.hip.add"],
                    "lowered_from": "serve.linear+serve.add",
                },
            )
            _replace(function, [l_index, a_index], a_index, new)
            return new.name
    return None


def _fuse_rope_store(function: Function) -> str | None:
    ops = function.block.operations
    uses, producer = _uses(function), _producers(function)
    for s_index, store in enumerate(ops):
        if store.name != "kernel.hip.kv_store" or len(store.operands) != 4:
            continue
        state, key, value, positions = store.operands
        r_index = producer.get(id(key))
        if r_index is None or ops[r_index].name != "kernel.hip.rope":
            continue
        rope = ops[r_index]
        if rope.results[1] is not key or not _only_used_by(uses, key, s_index):
            continue
        if len(uses[id(key)]) != 1:
            continue
        q_rot = rope.results[0]
        # The rotated query moves to the store's position: it must have no
        # user between the two.
        if any(user <= s_index for user, _ in uses[id(q_rot)]):
            continue
        q, k, cos, sin = rope.operands
        new = Operation(
            "kernel.hip.rope_kv_store",
            [state, q, k, value, cos, sin, positions],
            [q_rot, store.results[0]],
            {
                "slot": store.attributes.get("slot", 0),
                "head_dim": rope.attributes.get("head_dim"),
                "variant": rope.attributes.get("variant"),
                "fused_from": ["kernel.hip.rope", "kernel.hip.kv_store"],
                "lowered_from": "serve.rope+serve.kv.store",
            },
            store.effects,
        )
        _replace(function, [r_index, s_index], s_index, new)
        return new.name
    return None


def _fuse_store_advance(function: Function) -> str | None:
    """rope_kv_store whose state feeds only the kv.advance of the same slot
    (nothing reads the state in between), with positions = that slot's
    kv.length of the same incoming state: the store kernel advances too."""

    ops = function.block.operations
    uses, producer = _uses(function), _producers(function)
    for s_index, store in enumerate(ops):
        if store.name != "kernel.hip.rope_kv_store" or store.attributes.get("advance"):
            continue
        state_in, positions = store.operands[0], store.operands[6]
        p_index = producer.get(id(positions))
        if p_index is None:
            continue
        length = ops[p_index]
        if (length.name != "runtime.kv.length" or length.operands[0] is not state_in
                or length.attributes.get("slot", 0) != store.attributes.get("slot", 0)):
            continue
        state_out = store.results[1]
        users = uses[id(state_out)]
        if len(users) != 1 or users[0][0] >= len(ops):
            continue
        a_index = users[0][0]
        advance = ops[a_index]
        if (advance.name != "runtime.kv.advance"
                or advance.attributes.get("slot", 0) != store.attributes.get("slot", 0)):
            continue
        delta = int(advance.attributes.get("delta", 1))
        if delta <= 0:
            continue
        # The positions tensor is advanced in place when the state's lengths
        # are: nothing may read it after the store.
        if any(user > s_index for user, _ in uses[id(positions)]):
            continue
        attributes = dict(store.attributes)
        attributes["advance"] = delta
        attributes["fused_from"] = list(store.attributes.get("fused_from", [store.name])) + [advance.name]
        attributes["lowered_from"] = str(store.attributes.get("lowered_from", "")) + "+serve.kv.advance"
        new = Operation(store.name, list(store.operands), [store.results[0], advance.results[0]],
                        attributes, store.effects)
        _replace(function, [s_index, a_index], a_index, new)
        return "kernel.hip.rope_kv_store+advance"
    return None


def _fuse_store_attention(function: Function) -> str | None:
    """rope_kv_store advancing by one token whose rotated query and advanced
    state feed a decode_attention of the same slot (the query nowhere else,
    nothing touching either state in between): one kernel stores, advances
    and attends."""

    ops = function.block.operations
    uses = _uses(function)
    for s_index, store in enumerate(ops):
        if store.name != "kernel.hip.rope_kv_store" or store.attributes.get("advance") != 1:
            continue
        q_rot, state_out = store.results
        users = uses[id(q_rot)]
        if len(users) != 1 or users[0][0] >= len(ops) or users[0][1] != 1:
            continue
        a_index = users[0][0]
        attention = ops[a_index]
        # An attention with a profile-planned split keeps its own launch (the
        # fused kernel runs the fixed-chunk split only).
        if (attention.name != "kernel.hip.decode_attention" or len(attention.operands) != 3
                or attention.operands[0] is not state_out
                or attention.attributes.get("slot", 0) != store.attributes.get("slot", 0)
                or "split_plan" in attention.attributes):
            continue
        state_in = store.operands[0]
        between = range(s_index + 1, a_index)
        if any(user in between for value in (state_in, state_out) for user, _ in uses[id(value)]):
            continue
        attributes = {
            "slot": store.attributes.get("slot", 0),
            "head_dim": store.attributes.get("head_dim"),
            "variant": store.attributes.get("variant"),
            "advance": 1,
            "groups": attention.attributes["groups"],
            "scale": attention.attributes["scale"],
            "algorithm": attention.attributes.get("algorithm"),
            "numerical_mode": attention.attributes.get("numerical_mode"),
            "softmax_order": attention.attributes.get("softmax_order", "online"),
            "fused_from": list(store.attributes.get("fused_from", [store.name])) + [attention.name],
            "lowered_from": str(store.attributes.get("lowered_from", "")) + "+serve.decode_attention",
        }
        new = Operation("kernel.hip.rope_store_attention",
                        list(store.operands) + [attention.operands[2]],
                        [attention.results[0], state_out], attributes, store.effects)
        _replace(function, [s_index, a_index], a_index, new)
        return new.name
    return None
