"""Shared cases for the Zennit-compatible affine LRP rules (src/lrp_rules.cpp:72-160): the known
answers of a one-output layer, the Zennit 1.0.0 MLP of tests/lrp_reference_test.cpp:285-303, and a
float64 per-element statement of each rule's definition (the Zennit formulas term by term), used
as an independent check of the GEMM-composed implementations.

Test infrastructure only.
"""
import json
import os

import numpy as np

import oracle_ctypes as oc
from hf_fixtures import GOLDEN, det

E, G, AB, ZB = oc.EPSILON, oc.GAMMA, oc.ALPHA_BETA, oc.ZBOX


def rule(kind, **kw):
    return oc.lrp_rule(kind, **kw)


def eps_bias(eps=1e-6):
    return oc.lrp_rule(E, epsilon=eps, bias_in_denominator=True)


# One output: W = [1, -2, -1]^T, b = 0.5, x = [2, -1, 1], R = 1, so xW = 3 and z = 3.5; and the
# negative-output layer W = [-1, 1, 0.5]^T, b = -0.5, x = [2, -1, 1], R = 2, z = -3. Each expected
# vector is worked out by hand from the rule's definition:
#  * epsilon, bias in z:  x_i W_i / z = [2, 2, -1] / 3.5; pre-bias: [2, 2, -1] / 3
#  * ZPlus (AlphaBeta 1, 0): z+ = x+W+ (2) + b+ (0.5) + x-W- (2) = 4.5, shares [2, 2, 0] / 4.5
#  * AlphaBeta(2, 1): z- = x+W- = -1, negative shares [0, 0, -1]: 2 [2, 2, 0] / 4.5 - [0, 0, -1] / -1
#  * Gamma(0.5): Wa = [1.5, -2, -1], Wb = [1, -3, -1.5], ba = 0.75; z > 0 so the positive pair:
#    den = x+Wa + ba + x-Wb = 2.75 + 3 = 5.75, shares (x+ Wa + x- Wb) = [3, 3, -1]
#  * Gamma(0.5), z < 0: Wa = [-1, 1.5, 0.75], Wb = [-1.5, 1, 0.5], bb = -0.75;
#    den = x+Wb + bb + x-Wa = -3.25 - 1.5 = -4.75, shares (x+ Wb + x- Wa) = [-3, -1.5, 0.5], times R = 2
#  * ZBox(-1, 2): den = xW - L W+ - H W- = 3 + 1 + 6 = 10, shares [2, 2, -1] - [-1, 0, 0] - [0, -4, -2]
SINGLE_X = np.array([[2.0, -1.0, 1.0]], np.float32)
SINGLE_W = np.array([[1.0], [-2.0], [-1.0]], np.float32)
SINGLE_B = np.array([0.5], np.float32)
SINGLE_CASES = [
    ("epsilon bias in z", eps_bias(), [2 / 3.5, 2 / 3.5, -1 / 3.5]),
    ("epsilon pre-bias", oc.lrp_rule(E), [2 / 3, 2 / 3, -1 / 3]),
    ("zplus", rule(AB, alpha=1.0, beta=0.0), [2 / 4.5, 2 / 4.5, 0.0]),
    ("alpha2beta1", rule(AB, alpha=2.0, beta=1.0), [4 / 4.5, 4 / 4.5, -1.0]),
    ("gamma 0.5", rule(G, gamma=0.5), [3 / 5.75, 3 / 5.75, -1 / 5.75]),
    ("zbox -1 2", rule(ZB, low=-1.0, high=2.0), [0.3, 0.6, 0.1]),
]
NEG_W = np.array([[-1.0], [1.0], [0.5]], np.float32)
NEG_B = np.array([-0.5], np.float32)
NEG_R = np.array([[2.0]], np.float32)
NEG_EXPECTED = [-3 * 2 / -4.75, -1.5 * 2 / -4.75, 0.5 * 2 / -4.75]

# The reference's batch layer (lrp_rules_test.cpp): 4 -> 3, batch 2, mixed signs, no near-zero outputs.
BATCH_X = np.array([1.0, -2.0, 0.5, 3.0, -1.5, 0.25, 2.0, -0.75], np.float32).reshape(2, 4)
BATCH_W = np.array([0.5, -1.0, 0.75, -0.25, 2.0, -1.5, 1.25, 0.5, -0.5, -0.75, 0.25, 1.0], np.float32).reshape(4, 3)
BATCH_B = np.array([0.3, -0.2, 0.1], np.float32)
BATCH_R = np.array([1.0, -0.5, 2.0, 0.25, 1.5, -1.0], np.float32).reshape(2, 3)


def all_rules():
    return [("epsilon bias", eps_bias()), ("zplus", rule(AB, alpha=1.0, beta=0.0)),
            ("alpha2beta1", rule(AB, alpha=2.0, beta=1.0)), ("gamma 0.25", rule(G, gamma=0.25)),
            ("zbox -1.5 2", rule(ZB, low=-1.5, high=2.0))]


def rule_by_definition(x, w, b, r, c):
    """The rule's input relevance in float64, term by term from its definition (Zennit 1.0.0
    rules.py, as lrp_rules.hpp:6-21 states them): contribution of input i to output j, summed over j."""
    x, w, r = (np.asarray(a, np.float64) for a in (x, w, r))
    b = np.zeros(w.shape[1]) if b is None else np.asarray(b, np.float64)
    eps = float(np.float32(c.epsilon))
    stab = lambda v: v + eps * np.where(v >= 0, 1.0, -1.0)  # noqa: E731
    pos, neg = (lambda v: np.maximum(v, 0.0)), (lambda v: np.minimum(v, 0.0))
    X, W = x[:, :, None], w[None, :, :]  # (n, in, 1), (1, in, out)
    z = (X * W).sum(1) + b  # (n, out)
    if c.rule == E:
        zz = z if c.bias_in_denominator else z - b
        contrib = X * W * (r / stab(zz))[:, None, :]
    elif c.rule == AB:
        pp = pos(X) * pos(W) + neg(X) * neg(W)
        nn = pos(X) * neg(W) + neg(X) * pos(W)
        zp, zn = pp.sum(1) + pos(b), nn.sum(1) + neg(b)
        contrib = c.alpha * pp * (r / stab(zp))[:, None, :] - c.beta * nn * (r / stab(zn))[:, None, :]
    elif c.rule == G:
        g = float(np.float32(c.gamma))
        wa, wb = W + g * pos(W), W + g * neg(W)
        ba, bb = b + g * pos(b), b + g * neg(b)
        tp, tn = pos(X) * wa + neg(X) * wb, pos(X) * wb + neg(X) * wa
        dp, dn = tp.sum(1) + ba, tn.sum(1) + bb
        contrib = (np.where(z > 0, r / stab(dp), 0.0)[:, None, :] * tp +
                   np.where(z < 0, r / stab(dn), 0.0)[:, None, :] * tn)
    else:
        lo, hi = float(np.float32(c.low)), float(np.float32(c.high))
        t = X * W - lo * pos(W) - hi * neg(W)
        contrib = t * (r / stab(t.sum(1)))[:, None, :]
    return contrib.sum(2)


def zennit_values():
    return json.load(open(os.path.join(GOLDEN, "zennit_values.json")))


# Linear(6,8) -> ReLU -> Linear(8,5) -> ReLU -> Linear(5,3), every parameter det(...), input (2, 6)
# det(12, 5, 3, 5), one-hot targets {2, 1} (lrp_reference_test.cpp:285-303; weights (in, out)).
MLP_LAYERS = [(6, 8, 5, 1, 7, 2, 11), (8, 5, 3, 1, 9, 6, 13), (5, 3, 13, 1, 6, 10, 7)]
MLP_TARGETS = (2, 1)


def mlp_params():
    out = []
    for i, o, mul, add, div, badd, bdiv in MLP_LAYERS:
        out.append((det(i * o, mul, add, div).reshape(i, o), det(o, 3, badd, bdiv)))
    return out


def mlp_input():
    return det(12, 5, 3, 5).reshape(2, 6)


def mlp_cases():
    """(name, rule, expected key) of the Zennit cases (ZennitCases, lrp_reference_test.cpp:262-279). On
    this Conv-free MLP the three presets are Epsilon(1e-6) on every layer."""
    return [("Epsilon(1e-6)", eps_bias(1e-6), "kMlpEpsilon1e6"), ("Epsilon(0.25)", eps_bias(0.25), "kMlpEpsilon025"),
            ("ZPlus", rule(AB, alpha=1.0, beta=0.0), "kMlpZPlus"),
            ("AlphaBeta(2,1)", rule(AB, alpha=2.0, beta=1.0), "kMlpAlphaBeta21"),
            ("Gamma(0.25)", rule(G, gamma=0.25), "kMlpGamma025"),
            ("EpsilonPlus", eps_bias(1e-6), "kMlpEpsilonPlus"),
            ("EpsilonAlpha2Beta1", eps_bias(1e-6), "kMlpEpsilonAlpha2Beta1"),
            ("EpsilonGammaBox(-3,3)", eps_bias(1e-6), "kMlpEpsilonGammaBox")]


def mlp_seed():
    seed = np.zeros((2, 3), np.float32)
    for n, t in enumerate(MLP_TARGETS):
        seed[n, t] = 1.0
    return seed


def expect_reference_close(actual, expected):
    """The reference's tolerance for these values: |a - e| <= 1e-4 max(1, |e|) (lrp_reference_test.cpp:85-91)."""
    expected = np.asarray(expected, np.float32).ravel()
    actual = np.asarray(actual, np.float32).ravel()
    assert actual.shape == expected.shape
    err = np.abs(actual - expected) - 1e-4 * np.maximum(1.0, np.abs(expected))
    assert np.all(err <= 0), "max excess %g at %d" % (err.max(), int(np.argmax(err)))
