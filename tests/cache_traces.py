"""Scripted expert-cache traces (test infrastructure): seeded sequences of the calls a MoE layer
makes on its Glm53fExpertSrc during decode (src/core/glm53f_ops.c:1190-1342): hint its own
experts and the next layer's predictions, get each unique expert, release them, with getmany
batches and background reads in between. Keys live in the reference's glm_tiny layout: 6 layers
(5 + the MTP layer), 6 routed experts, MoE layers 1-4, top-2."""
import random

N_LAYERS, N_EXPERTS, TOPK = 6, 6, 2
MOE_LAYERS = [1, 2, 3, 4]


def trace(seed, steps, nslot, with_hints=True, with_getmany=True):
    rnd = random.Random(seed)
    ops = []
    for _ in range(steps):
        for L in MOE_LAYERS:
            ids = rnd.sample(range(N_EXPERTS), TOPK)
            if with_hints:
                ops += [4, L, len(ids)] + ids
                if L + 1 in MOE_LAYERS:       # the checkpoint has no MTP layer (5)
                    pred = rnd.sample(range(N_EXPERTS), rnd.randint(1, 3))
                    ops += [4, L + 1, len(pred)] + pred
                ops += [5, rnd.randint(0, 3)]
            if with_getmany and rnd.random() < 0.3:
                ops += [3, L, len(ids)] + ids
            for e in ids:
                ops += [1, L, e]
            if rnd.random() < 0.2 and nslot > TOPK + 1:
                ops += [1, L, ids[0]]                 # a second pin of the same expert
                ops += [2, L, ids[0]]
            for e in ids:
                ops += [2, L, e]
    return ops


CASES = [  # (seed, steps, nslot, hints, getmany)
    (1, 6, 3, False, False),
    (2, 6, 3, True, False),
    (3, 8, 5, True, True),
    (4, 8, 10, True, True),
    (5, 10, 24, True, True),
    (6, 12, 4, False, True),
]
