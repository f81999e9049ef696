"""Input recipes of the five BASELINE configurations (synthetic, portable).

Every input comes from the oracle's SplitMix64-based generators (exact integer and
single-rounding float arithmetic only), so the same recipe gives the same bits on every
machine. Each case is a dict: name, M, N, K, ta, tb, S and a `make()` returning the
stored operands (A, B) as float32 arrays in the layouts the transposes imply:
A is MxK (KxM if ta), B is KxN (NxK if tb).
"""
import numpy as np

from oracle import oracle as O


def _case(name, M, N, K, ta, tb, S, make):
    return dict(name=name, M=M, N=N, K=K, ta=int(ta), tb=int(tb), S=S, make=make)


def config1():
    """256^3, S=3, no transposes; A then B N(0,1) from one stream, seed 12345
    (the order of repro_gemm_cuda/hash_repro_gemm.cu:93-94 with dist=normal)."""
    n = 256 * 256
    return [_case("c1.256cube", 256, 256, 256, 0, 0, 3,
                  lambda: (O.gen_normal(n, 1.0, 12345, 0), O.gen_normal(n, 1.0, 12345, n)))]


def _lenet_bound(fan_in):
    # float32 1 / sqrt(fan_in), as repro_torch/utils.py:40
    return float(np.float32(1.0) / np.sqrt(np.float32(fan_in)))


def config2():
    """LeNet-5 linear layers, batch 64, S = 1, 2, 3: forward Y = X W^T, dX = dY W,
    dW = dY^T X for 400->120, 120->84, 84->10. W ~ U(+-1/sqrt(fan_in)) (float32 recipe of
    repro_torch/utils.py:23-29); X, dY ~ N(0,1). Seeds 2024 + 100*layer + {1, 2, 3}."""
    cases = []
    for li, (fin, fout) in enumerate([(400, 120), (120, 84), (84, 10)]):
        s = 2024 + 100 * li
        X = lambda fin=fin, s=s: O.gen_normal(64 * fin, 1.0, s + 1)
        W = lambda fin=fin, fout=fout, s=s: O.gen_uniform_pm(fout * fin, _lenet_bound(fin), s + 2)
        dY = lambda fout=fout, s=s: O.gen_normal(64 * fout, 1.0, s + 3)
        tag = "c2.fc%d.%dx%d" % (li + 1, fin, fout)
        for S in (1, 2, 3):
            cases.append(_case(tag + ".fwd.S%d" % S, 64, fout, fin, 0, 1, S,
                               lambda X=X, W=W: (X(), W())))
            cases.append(_case(tag + ".dX.S%d" % S, 64, fin, fout, 0, 0, S,
                               lambda dY=dY, W=W: (dY(), W())))
            cases.append(_case(tag + ".dW.S%d" % S, fout, fin, 64, 1, 0, S,
                               lambda dY=dY, X=X: (dY(), X())))
    return cases


def config3():
    """GPT-2-small linear GEMMs at B*T = 8192 tokens, C = 768, S = 3: QKV 768->2304,
    attn-proj 768->768, MLP 768->3072 and 3072->768, each forward, dX and dW.
    W ~ N(0, 0.02); X, dY ~ N(0,1). Seeds 3000 + 10*j + {1, 2, 3}."""
    T = 8192
    cases = []
    for j, (nm, fin, fout) in enumerate([("qkv", 768, 2304), ("attn_proj", 768, 768),
                                         ("mlp_fc", 768, 3072), ("mlp_proj", 3072, 768)]):
        s = 3000 + 10 * j
        X = lambda fin=fin, s=s: O.gen_normal(T * fin, 1.0, s + 1)
        W = lambda fin=fin, fout=fout, s=s: O.gen_normal(fout * fin, 0.02, s + 2)
        dY = lambda fout=fout, s=s: O.gen_normal(T * fout, 1.0, s + 3)
        tag = "c3." + nm
        cases.append(_case(tag + ".fwd", T, fout, fin, 0, 1, 3, lambda X=X, W=W: (X(), W())))
        cases.append(_case(tag + ".dX", T, fin, fout, 0, 0, 3, lambda dY=dY, W=W: (dY(), W())))
        cases.append(_case(tag + ".dW", fout, fin, T, 1, 0, 3, lambda dY=dY, X=X: (dY(), X())))
    return cases


def config4():
    """Adversarial dynamic range, 4096^3, S = 3, no transposes. Random signs, |x| = 2^e
    with e ~ U[-60, 60], 5% exact zeros, 1% subnormals. Elements pair up along k: in A
    the second of each pair is the negated first times (1 + 2^-20 t), in B it is the first
    times (1 + 2^-20 t), so every dot product cancels almost exactly."""
    n = 4096
    return [_case("c4.adversarial4096", n, n, n, 0, 0, 3,
                  lambda: (O.gen_adversarial(n, n, 4001, pair_rows=False, negate=True),
                           O.gen_adversarial(n, n, 4002, pair_rows=True, negate=False)))]


def config5():
    """Large and skewed, S = 3, inputs N(0,1): GPT-2 LM-head forward M=8192, K=768,
    N=50257 (B^T); its dW M=50257, N=768, K=8192 (A^T); tall-skinny M=N=1024, K=65536."""
    return [
        _case("c5.lm_head.fwd", 8192, 50257, 768, 0, 1, 3,
              lambda: (O.gen_normal(8192 * 768, 1.0, 5001), O.gen_normal(50257 * 768, 1.0, 5002))),
        _case("c5.lm_head.dW", 50257, 768, 8192, 1, 0, 3,
              lambda: (O.gen_normal(8192 * 50257, 1.0, 5003), O.gen_normal(8192 * 768, 1.0, 5001))),
        _case("c5.tall_skinny", 1024, 1024, 65536, 0, 0, 3,
              lambda: (O.gen_normal(1024 * 65536, 1.0, 5004), O.gen_normal(65536 * 1024, 1.0, 5005))),
    ]


ALL = {1: config1, 2: config2, 3: config3, 4: config4, 5: config5}


def all_cases():
    out = []
    for k in sorted(ALL):
        out.extend(ALL[k]())
    return out
