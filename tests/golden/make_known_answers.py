"""Writes known_answers.json: tiny routing cases with their expected CSR and
permutation, derived here by brute force in pure Python (no oracle code).

The reference tree has no golden vectors for this path (it contains no MoE
code at all), so these known answers are derived from the specification's
definitions: score = 1 / (1 + exp(-logit)), routed iff score >= thr[e],
fallback to the first argmax expert, slots ordered by (expert, token id).
Logits are chosen far from every threshold (|score - thr| > 1e-3), so the
float64 sigmoid used here decides every comparison exactly as any
correctly-rounded binary32 sigmoid does.  Run: python tests/golden/make_known_answers.py
"""
import json
import math
import os

CASES = [
    # name, logits [T][E], thr [E]
    ("basic_3x4", [[2.0, -1.0, 0.5, 3.0],
                   [-2.0, -3.0, -1.5, -4.0],
                   [1.0, 1.0, -0.5, 0.0]], [0.7, 0.7, 0.55, 0.9]),
    ("all_fallback_ties", [[0.0, 0.0, -1.0],
                           [-2.0, 1.0, 1.0],
                           [-5.0, -5.0, -5.0]], [0.99, 0.99, 0.99]),
    ("single_expert", [[0.3], [-0.3], [5.0]], [0.6]),
    ("all_routed", [[-1.0, 0.0], [2.0, -2.0]], [0.0, 0.0]),
    ("skewed_5x3", [[4.0, -4.0, -4.0], [4.0, 0.2, -4.0], [4.0, -4.0, 0.4],
                    [-4.0, -4.0, -4.0], [4.0, 4.0, 4.0]], [0.6, 0.5, 0.58]),
]


def solve(logits, thr):
    T, E = len(logits), len(thr)
    score = [[1.0 / (1.0 + math.exp(-l)) for l in row] for row in logits]
    for t in range(T):
        for e in range(E):
            assert abs(score[t][e] - thr[e]) > 1e-3 or thr[e] == 0.0, (t, e)
    sel = [[score[t][e] >= thr[e] for e in range(E)] for t in range(T)]
    for t in range(T):
        if not any(sel[t]):
            best = max(range(E), key=lambda e: (score[t][e], -e))
            sel[t][best] = True
    pairs = [(e, t) for e in range(E) for t in range(T) if sel[t][e]]   # (expert, token) order
    counts = [sum(sel[t][e] for t in range(T)) for e in range(E)]
    eoff = [0]
    for c in counts:
        eoff.append(eoff[-1] + c)
    slot = {p: i for i, p in enumerate(pairs)}
    toff, tslot = [0], []
    for t in range(T):
        for e in range(E):
            if sel[t][e]:
                tslot.append(slot[(e, t)])
        toff.append(len(tslot))
    return dict(counts=counts, expert_offsets=eoff, token_offsets=toff,
                sorted_token=[t for _, t in pairs], token_slot=tslot,
                slot_expert=[e for e, _ in pairs])


def main():
    out = []
    for name, logits, thr in CASES:
        out.append(dict(name=name, logits=logits, thr=thr, expected=solve(logits, thr)))
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "known_answers.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print("wrote", path)


if __name__ == "__main__":
    main()
