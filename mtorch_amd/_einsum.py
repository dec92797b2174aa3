"""einsum over device tensors, lowered onto the batched GEMM.

The reference dispatches einsum in two steps (mtorch/__init__.py:1063-1140): its native
`_C.einsum` recognises the attention equations -- "ij,jk", "...ij,...jk->...ik",
"bij,bjk->bik", "bhij,bhjd->bhid" and, for a shared prefix, "PREFIXij,PREFIXjk->PREFIXik" and
"PREFIXid,PREFIXjd->PREFIXij" (module.cpp:6282-6365) -- as matmul(l, r) and
matmul(l, r.transpose(-1, -2)); anything else goes through its Python label algebra
(permute, broadcast multiply, sum).  Here every equation whose contractions can be written as
products is planned as label groups instead:

    batch    -- in both operands and in the output      -> the GEMM batch
    left     -- in the left operand and the output only  -> GEMM rows
    right    -- in the right operand and the output only -> GEMM columns
    contract -- in both operands, not in the output      -> GEMM depth

Each operand is permuted (a view) to (batch, left, contract) / (batch, contract, right), folded to
three dims (a view where the strides allow it, else one gather copy), multiplied by the MFMA
GEMM, and the result is unfolded and permuted to the output order.  The native patterns above are
the special cases with empty batch/left/right groups.  Three or more operands are contracted left
to right, keeping the labels a later operand or the output still needs.

Equations this lowering cannot express as products raise NotImplementedError: a label repeated
inside one operand (a diagonal) and a label summed within one operand alone (a reduction).
"""

from __future__ import annotations

from . import _ops
from . import _tensor as T

_ELLIPSIS = "..."


def _parse(spec: str):
    tokens, i, seen_ellipsis = [], 0, False
    while i < len(spec):
        if spec.startswith(_ELLIPSIS, i):
            if seen_ellipsis:
                raise ValueError("einsum subscript contains more than one ellipsis")
            tokens.append(_ELLIPSIS)
            seen_ellipsis = True
            i += 3
            continue
        ch = spec[i]
        if not ch.isalpha():
            raise ValueError(f"einsum subscript contains invalid character '{ch}'")
        tokens.append(ch)
        i += 1
    return tokens


def _expand(tokens, rank, ellipsis_labels):
    explicit = sum(1 for t in tokens if t is not _ELLIPSIS)
    if _ELLIPSIS not in tokens:
        if explicit != rank:
            raise ValueError("einsum subscript rank does not match operand rank")
        return list(tokens)
    n = rank - explicit
    if n < 0:
        raise ValueError("einsum subscript rank does not match operand rank")
    labels = []
    for t in tokens:
        if t is _ELLIPSIS:
            labels.extend(ellipsis_labels[len(ellipsis_labels) - n:] if n else [])
        else:
            labels.append(t)
    return labels


def _prod(sizes):
    n = 1
    for s in sizes:
        n *= s
    return n


def _fold(t: T.Tensor, labels, groups, sizes):
    """Permute t (labelled `labels`) to the concatenation of `groups`, broadcast size-1 dims to
    `sizes`, and fold each group to one dim."""
    order = [labels.index(l) for g in groups for l in g]
    p = t.permute(order) if order != list(range(len(order))) else t
    target = [sizes[l] for g in groups for l in g]
    if list(p.shape) != target:
        p = p.expand(target)
    return p.reshape([_prod([sizes[l] for l in g]) for g in groups])


def _contract(a, la, b, lb, keep, sizes):
    """Contract two labelled operands, keeping the labels in `keep`; returns (tensor, labels)."""
    in_b = set(lb)
    in_a = set(la)
    batch = [l for l in la if l in in_b and l in keep]
    contract = [l for l in la if l in in_b and l not in keep]
    left = [l for l in la if l not in in_b]
    right = [l for l in lb if l not in in_a]
    for side, group in (("left", left), ("right", right)):
        summed = [l for l in group if l not in keep]
        if summed:
            raise NotImplementedError(
                f"mtorch_amd: einsum label(s) {''.join(summed)} are summed within the {side} operand alone (a "
                "reduction); only contractions that lower onto the GEMM are implemented")
    a3 = _fold(a, la, (batch, left, contract), sizes)
    b3 = _fold(b, lb, (batch, contract, right), sizes)
    out_sizes = [sizes[l] for l in batch + left + right]
    if _prod([sizes[l] for l in contract]) == 0:
        out = _ops._empty(out_sizes, a.dtype, a._dev())
        _ops.fill_(out, 0.0)
        return out, batch + left + right
    c = _ops.matmul(a3, b3)
    return c.reshape(out_sizes), batch + left + right


def einsum(equation, *operands):
    """mtorch.einsum (mtorch/__init__.py:1063; native patterns module.cpp:6282-6365)."""
    if len(operands) == 1 and isinstance(operands[0], (list, tuple)):
        operands = tuple(operands[0])
    if not isinstance(equation, str):
        raise TypeError("einsum equation must be a string")
    if not operands:
        raise ValueError("einsum expected at least one operand")
    compact = equation.replace(" ", "")
    if "->" in compact:
        inputs_text, output_text = compact.split("->", 1)
        explicit_output = True
    else:
        inputs_text, output_text, explicit_output = compact, "", False
    specs = inputs_text.split(",")
    if len(specs) != len(operands):
        raise ValueError("einsum operand count does not match equation")
    parsed = [_parse(s) for s in specs]
    ell_rank = 0
    for tokens, op in zip(parsed, operands):
        ell_rank = max(ell_rank, op.dim() - sum(1 for t in tokens if t is not _ELLIPSIS))
    ellipsis_labels = [f"@{i}" for i in range(ell_rank)]

    labels_by_op, sizes, counts = [], {}, {}
    for tokens, op in zip(parsed, operands):
        labels = _expand(tokens, op.dim(), ellipsis_labels)
        if len(set(labels)) != len(labels):
            raise NotImplementedError("mtorch_amd: einsum with a label repeated inside one operand (a diagonal) "
                                      "is not implemented")
        for l, s in zip(labels, op.shape):
            if l in sizes and sizes[l] != s:
                if sizes[l] == 1:
                    sizes[l] = s
                elif s != 1:
                    raise ValueError(f"einsum label '{l}' has inconsistent sizes {sizes[l]} and {s}")
            else:
                sizes.setdefault(l, s)
            counts[l] = counts.get(l, 0) + 1
        labels_by_op.append(labels)

    if explicit_output:
        out_labels = []
        for t in _parse(output_text):
            out_labels.extend(ellipsis_labels if t is _ELLIPSIS else [t])
        if len(set(out_labels)) != len(out_labels):
            raise ValueError("einsum output subscript repeats a label")
        for l in out_labels:
            if l not in sizes:
                raise ValueError(f"einsum output label '{l}' does not appear in the inputs")
    else:
        out_labels = ellipsis_labels + sorted(l for l, c in counts.items() if c == 1 and not l.startswith("@"))

    dt = operands[0].dtype
    for op in operands:
        if op.dtype is not dt:
            raise ValueError("einsum operands must have the same dtype")
    _ops._gpu("einsum", *operands)

    cur, cur_labels = operands[0], labels_by_op[0]
    if len(operands) == 1:
        summed = [l for l in cur_labels if l not in out_labels]
        if summed:
            raise NotImplementedError("mtorch_amd: einsum reductions over one operand are not implemented")
    for k in range(1, len(operands)):
        keep = set(out_labels)
        for later in labels_by_op[k + 1:]:
            keep.update(later)
        cur, cur_labels = _contract(cur, cur_labels, operands[k], labels_by_op[k], keep, sizes)
    order = [cur_labels.index(l) for l in out_labels]
    if list(cur.shape) != [sizes[l] for l in cur_labels]:
        cur = cur.expand([sizes[l] for l in cur_labels])
    return cur.permute(order) if order != list(range(len(order))) else cur
