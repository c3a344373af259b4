"""Cases shared by the drop-in tests: the Zennit MLP of tests/lrp_reference_test.cpp:285-303 run
through the reference's own LRP::explain, with its uniform rules and the three composite presets."""
import rules_cases as rc

# (name, rule, preset, expected key): preset 0 = the uniform rule on every module, 1-3 = the
# reference's LRP::epsilon_plus(), epsilon_alpha2_beta1(), epsilon_gamma_box(-3, 3) (lrp.hpp:186-197).
PRESETS = {"EpsilonPlus": 1, "EpsilonAlpha2Beta1": 2, "EpsilonGammaBox(-3,3)": 3}


def explain_cases():
    return [(name, rule, PRESETS.get(name, 0), key) for name, rule, key in rc.mlp_cases()]
