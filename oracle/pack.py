"""CPU ORACLE -- test infrastructure only (see oracle/__init__.py).

Restatement of the ragged-batch packing: rows of one sequence form a
contiguous group (BatchItem runs of sched_iteration_joint, reference
examples/intfer_cli/main.cpp:8438-8488); each group is cut into q-blocks of
`qb` tokens; each q-block x kv head x KV split of `split` tokens is one
attention unit.  Pure Python loops over small batches.
"""


def pack(rows, nkv, qb, split):
    M = len(rows)
    starts = [m for m in range(M) if m == 0 or rows[m][0] != rows[m - 1][0]]
    cu = starts + [M]
    row_grp = []
    for g in range(len(starts)):
        row_grp += [g] * (cu[g + 1] - cu[g])
    units, comb_base, comb_nsplit, comb_tok = [], [0] * M, [0] * M, [0] * M
    for g in range(len(starts)):
        r0, n = cu[g], cu[g + 1] - cu[g]
        seq, pos0 = rows[r0][0], rows[r0][1]
        for b in range((n + qb - 1) // qb):
            qn = min(qb, n - b * qb)
            kvhi = pos0 + b * qb + qn
            ns = (kvhi + split - 1) // split
            base = len(units)
            for kvh in range(nkv):
                for s in range(ns):
                    units.append([seq, kvh, r0 + b * qb, qn, pos0 + b * qb, s * split,
                                  min((s + 1) * split, kvhi), 0])
            for i in range(qn):
                m = r0 + b * qb + i
                comb_base[m], comb_nsplit[m], comb_tok[m] = base, ns, i
    return {"cu_seqlens": cu, "row_grp": row_grp, "units": units, "comb_base": comb_base,
            "comb_nsplit": comb_nsplit, "comb_tok": comb_tok,
            "order": attn_order(rows, nkv, qb, split)}


def attn_order(rows, nkv, qb, split):
    """Attention dispatch slots (4 per workgroup): for groups with several
    q-blocks, chunks of 4 consecutive q-blocks share a workgroup per
    (kv head, split); then the units of single-q-block groups, densely.
    Unit ids follow pack()'s unit order."""
    M = len(rows)
    starts = [m for m in range(M) if m == 0 or rows[m][0] != rows[m - 1][0]]
    cu = starts + [M]
    chunked, dense, uid = [], [], 0
    for g in range(len(starts)):
        n, pos0 = cu[g + 1] - cu[g], rows[cu[g]][1]
        nb = (n + qb - 1) // qb
        ns = [(pos0 + min((b + 1) * qb, n) + split - 1) // split for b in range(nb)]
        base = []
        for b in range(nb):
            base.append(uid)
            uid += nkv * ns[b]
        if nb == 1:
            dense += list(range(base[0], base[0] + nkv * ns[0]))
            continue
        for j in range(0, nb, 4):
            blocks = list(range(j, min(j + 4, nb)))
            nsm = ns[blocks[-1]]
            for kvh in range(nkv):
                for s in range(nsm):
                    for q in range(4):
                        b = j + q
                        ok = b < nb and s < ns[b]
                        chunked.append(base[b] + kvh * ns[b] + s if ok else -1)
    return chunked + dense
