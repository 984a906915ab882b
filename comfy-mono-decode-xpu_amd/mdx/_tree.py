"""Draft-tree bookkeeping on the host: the tree_spec shape (a chain with leaf siblings at each depth,
the first child of a node being the chain), parents / children / depths in tree order, and the
verify program of the Gated-DeltaNet replay (comfy_mono_decode_xpu/mtp_loop.py:80-95 builds the
same tables from ComfyUI's VerifyTree)."""
from __future__ import annotations


def spec_of_widths(widths):
    """Nested child lists of tree_spec(widths): depth d has widths[d] children of the chain node."""
    node = []
    for w in reversed(widths):
        node = [node] + [[] for _ in range(w - 1)]
    return node


def tree_from_spec(spec, rows):
    """parents, children, depths (tree order: depth-first, chain child first), padded to `rows`, and
    the index of the chain's last node."""
    parent, children, depth = [], [], []
    stack = [(spec, -1)]
    while stack:
        node, p = stack.pop()
        r = len(parent)
        parent.append(p)
        children.append([])
        depth.append(0 if p < 0 else depth[p] + 1)
        if p >= 0:
            children[p].append(r)
        stack.extend((child, r) for child in reversed(node))
    end = 0
    while children[end]:
        end = children[end][0]
    while len(parent) < rows:
        parent.append(-1)
        children.append([])
        depth.append(0)
    return parent, children, depth, end


def verify_program(parents, rows):
    """Entries in an order where each row sees the recurrent state after exactly its ancestors: a
    chain node (committing, bit 32), then its leaf siblings (not committing), down the chain; the last
    entry need not commit. Returns the program (slot | commit) per entry."""
    children = [[] for _ in range(rows)]
    for r in range(rows):
        if parents[r] >= 0:
            children[parents[r]].append(r)
    order, node = [], 0
    while True:
        order.append([node, 32])
        kids = children[node]
        for leaf in kids[1:]:
            if children[leaf]:
                raise ValueError("only the first child of a node may have children")
            order.append([leaf, 0])
        if not kids:
            break
        node = kids[0]
    if order[-1][0] == node:
        order[-1][1] = 0
    if len(order) != rows:
        raise ValueError("the program must cover every row")
    return [n | c for n, c in order]
