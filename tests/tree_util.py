"""Seeded draft-tree shapes shared by the tree tests."""
import numpy as np


def random_tree(rng, n, branch=3, depth=5):
    """Parent array of n nodes: node i > 0 hangs below an earlier node of
    depth < depth with fewer than `branch` children; node 0 is the root."""
    parent, dep, kids = [-1], [0], [0]
    for i in range(1, n):
        ok = [v for v in range(i) if dep[v] < depth and kids[v] < branch]
        v = int(rng.choice(ok))
        parent.append(v)
        dep.append(dep[v] + 1)
        kids[v] += 1
        kids.append(0)
    return np.array(parent, np.int32)


def path_to(parent, i):
    """Nodes from the root to node i."""
    p = []
    while i >= 0:
        p.append(int(i))
        i = parent[i]
    return p[::-1]
