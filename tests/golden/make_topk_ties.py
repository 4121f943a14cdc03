"""Write the torch.topk tie table for groups of 4 (k = 1, 2, 3) as a JSON fixture.

The reference selects the kept members of every N:M group with
``torch.topk(view(out, in/M, M), k=N, dim=-1).indices`` followed by a scatter
(legacy/sparse_modeling.py:597-599 for nm_2_4, :730-734 for structured,
:1206-1208 for the beta mix, :1373-1376 for the nm_2_4 penalty target).  Which
members survive a tie is a property of torch's CPU topk, not of the
reference, so the table is produced here by calling torch.topk on every weak
ordering of four values (75 of them) and is committed as data.

Key of a group (v0, v1, v2, v3): lt_i = #{j : v_j < v_i}; key = sum lt_i << 2i.
Two groups have the same key exactly when they have the same weak ordering,
so the key indexes a 256-entry lookup table (75 entries are reachable).

Run:  python tests/golden/make_topk_ties.py
"""
import itertools
import json
import os

import torch


def group_key(vals):
    return sum(sum(1 for y in vals if y < x) << (2 * i) for i, x in enumerate(vals))


def main():
    out = {"torch_version": torch.__version__, "tables": {}}
    for k in (1, 2, 3):
        rows = {}
        for r in itertools.product(range(4), repeat=4):
            t = torch.tensor(r, dtype=torch.float32).view(1, 1, 4)
            idx = sorted(torch.topk(t, k, dim=-1).indices.view(-1).tolist())
            key = group_key(r)
            keep = sum(1 << i for i in idx)
            if key in rows:
                assert rows[key]["keep"] == keep
                continue
            rows[key] = {"pattern": list(r), "keep": keep}
        out["tables"][str(k)] = {str(key): v for key, v in sorted(rows.items())}
    path = os.path.join(os.path.dirname(__file__), "topk_ties_m4.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=0, sort_keys=True)
    print("wrote", path, {k: len(v) for k, v in out["tables"].items()})


if __name__ == "__main__":
    main()
