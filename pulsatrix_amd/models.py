"""Python handles over the host framework's C ABI (include/pulsatrix_amd.h).

Block and CausalLM take host numpy arrays (the parity-test interface, same calls as the oracle's
ctypes wrapper); CausalLM.explain_device runs the device hot path on buffers already in HBM.
"""
import ctypes

import numpy as np

from . import native as N


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def param_count(cfg, block=False):
    h = N.host()
    return (h.pxa_block_param_count if block else h.pxa_param_count)(ctypes.byref(cfg))


def synthetic_params(cfg, seed, std=0.02, block=False):
    """Random-init blob: N(0, std) from seed, every RMSNorm gamma 1 (SplitMix64 + Box-Muller)."""
    out = np.empty(param_count(cfg, block), np.float32)
    N.host_check(N.host().pxa_synthetic_params(ctypes.byref(cfg), int(block), seed, std, _p(out)))
    return out


def linear_relevance_rule(x, w, b, r, rule):
    """A LinearModule on the device: forward of x (n, in) through w (in, out) and bias b (nullable),
    then propagate_relevance of r (n, out) under `rule`. Returns (y, r_in)."""
    x, w, r = (np.ascontiguousarray(a, dtype=np.float32) for a in (x, w, r))
    b = None if b is None else np.ascontiguousarray(b, dtype=np.float32)
    n, i = x.shape
    o = w.shape[1]
    y = np.empty((n, o), np.float32)
    r_in = np.empty((n, i), np.float32)
    N.host_check(N.host().pxa_linear_relevance_rule(_p(x), _p(w), _p(b), n, i, o, _p(r), ctypes.byref(N.as_rule(rule)),
                                                    _p(y), _p(r_in)))
    return y, r_in


class Block:
    """TransformerBlock on the process-wide MI355XBackend."""

    def __init__(self, cfg, params):
        self.cfg = cfg
        params = np.ascontiguousarray(params, dtype=np.float32)
        self.h = N.host().pxa_block_create(ctypes.byref(cfg), _p(params))
        if not self.h:
            raise N.PxkError(N.host().pxa_last_error().decode())

    def forward(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        n, l, _ = x.shape
        y = np.empty_like(x)
        N.host_check(N.host().pxa_block_forward(self.h, _p(x), n, l, _p(y)))
        return y

    def relevance(self, r, eps, bias_in_denominator):
        r = np.ascontiguousarray(r, dtype=np.float32)
        out = np.empty_like(r)
        N.host_check(N.host().pxa_block_relevance(self.h, _p(r), eps, int(bias_in_denominator), _p(out)))
        return out

    def relevance_rule(self, r, rule):
        r = np.ascontiguousarray(r, dtype=np.float32)
        out = np.empty_like(r)
        N.host_check(N.host().pxa_block_relevance_rule(self.h, _p(r), ctypes.byref(N.as_rule(rule)), _p(out)))
        return out

    def __del__(self):
        if getattr(self, "h", None):
            N.host().pxa_block_destroy(self.h)
            self.h = None


class CausalLM:
    """CausalLM on the process-wide MI355XBackend."""

    def __init__(self, cfg, params=None, seed=None, std=0.02):
        self.cfg = cfg
        h = N.host()
        if params is None:
            self.h = h.pxa_lm_create_random(ctypes.byref(cfg), seed, std)
        else:
            params = np.ascontiguousarray(params, dtype=np.float32)
            self.h = h.pxa_lm_create(ctypes.byref(cfg), _p(params))
        if not self.h:
            raise N.PxkError(h.pxa_last_error().decode())
        self.shape = None

    @classmethod
    def load(cls, directory):
        """LoadCausalLM: a Hugging Face checkpoint directory, weights converted on the device."""
        self = cls.__new__(cls)
        cfg = N.ModelConfig()
        self.h = N.host().pxa_lm_load(str(directory).encode(), ctypes.byref(cfg))
        if not self.h:
            raise N.PxkError(N.host().pxa_last_error().decode())
        self.cfg, self.shape = cfg, None
        return self

    def forward(self, ids):
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        n, l = ids.shape
        logits = np.empty((n, l, self.cfg.vocab_size), np.float32)
        N.host_check(N.host().pxa_lm_forward(self.h, ids.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)), n, l,
                                             _p(logits)))
        self.shape = (n, l)
        return logits

    def _relevance_outputs(self, want_kv):
        n, l = self.shape
        c = self.cfg
        kvh = c.num_kv_heads if c.num_kv_heads > 0 else c.num_heads
        hd = c.head_dim if c.head_dim > 0 else c.hidden_size // c.num_heads
        kv = (c.num_layers, n * l, kvh * hd)
        return (np.empty((n, l, c.hidden_size), np.float32), np.empty((n, l), np.float32),
                np.empty(kv, np.float32) if want_kv else None, np.empty(kv, np.float32) if want_kv else None)

    def relevance(self, seed, eps, bias_in_denominator, want_kv=False):
        seed = np.ascontiguousarray(seed, dtype=np.float32)
        r_embed, r_tok, k, v = self._relevance_outputs(want_kv)
        N.host_check(N.host().pxa_lm_relevance(self.h, _p(seed), eps, int(bias_in_denominator), _p(r_embed),
                                               _p(r_tok), _p(k), _p(v)))
        return (r_embed, r_tok, k, v) if want_kv else (r_embed, r_tok)

    def relevance_rule(self, seed, rule, want_kv=False):
        """propagate_relevance_by_layer under any LRPRuleConfig (an LrpRule, or the oracle's)."""
        seed = np.ascontiguousarray(seed, dtype=np.float32)
        r_embed, r_tok, k, v = self._relevance_outputs(want_kv)
        N.host_check(N.host().pxa_lm_relevance_rule(self.h, _p(seed), ctypes.byref(N.as_rule(rule)), _p(r_embed),
                                                    _p(r_tok), _p(k), _p(v)))
        return (r_embed, r_tok, k, v) if want_kv else (r_embed, r_tok)

    def explain_device(self, ids_ptr, n, l, eps, bias_in_denominator, token_rel_ptr, targets_ptr, targets=None,
                       unit_seed=False):
        """Device hot path; pointers are device addresses (ints or c_void_p)."""
        t = None
        if targets is not None:
            t = np.ascontiguousarray(targets, dtype=np.int64)
        N.host_check(N.host().pxa_lm_explain_device(
            self.h, ids_ptr, n, l, eps, int(bias_in_denominator), token_rel_ptr, targets_ptr,
            t.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)) if t is not None else None, int(unit_seed)))

    def capture_explain(self, ids_ptr, n, l, eps, bias_in_denominator, token_rel_ptr, targets_ptr):
        N.host_check(N.host().pxa_lm_capture_explain(self.h, ids_ptr, n, l, eps, int(bias_in_denominator),
                                                     token_rel_ptr, targets_ptr))

    def explain_device_rule(self, ids_ptr, n, l, rule, token_rel_ptr, targets_ptr, targets=None, unit_seed=False):
        t = None if targets is None else np.ascontiguousarray(targets, dtype=np.int64)
        N.host_check(N.host().pxa_lm_explain_device_rule(
            self.h, ids_ptr, n, l, ctypes.byref(N.as_rule(rule)), token_rel_ptr, targets_ptr,
            t.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)) if t is not None else None, int(unit_seed)))

    def capture_explain_rule(self, ids_ptr, n, l, rule, token_rel_ptr, targets_ptr):
        N.host_check(N.host().pxa_lm_capture_explain_rule(self.h, ids_ptr, n, l, ctypes.byref(N.as_rule(rule)),
                                                          token_rel_ptr, targets_ptr))

    def explain_rows_device(self, ids_ptr, n, l, targets_ptr, target_stride, rule, token_rel_ptr, targets_out_ptr=None,
                            unit_seed=False):
        N.host_check(N.host().pxa_lm_explain_rows_device(self.h, ids_ptr, n, l, targets_ptr, target_stride,
                                                         ctypes.byref(N.as_rule(rule)), token_rel_ptr, targets_out_ptr,
                                                         int(unit_seed)))

    def generate_device(self, ids_ptr, n, prompt, new_tokens, ld_ids, picked_logit_ptr=None):
        """Batched KV-cached greedy decode into the id rows (device pointers)."""
        N.host_check(N.host().pxa_lm_generate_device(self.h, ids_ptr, n, prompt, new_tokens, ld_ids, picked_logit_ptr))

    def explain_generated_device(self, ids_ptr, n, prompt, new_tokens, ld_ids, rule, token_rel_ptr, unit_seed=False):
        N.host_check(N.host().pxa_lm_explain_generated_device(self.h, ids_ptr, n, prompt, new_tokens, ld_ids,
                                                              ctypes.byref(N.as_rule(rule)), token_rel_ptr,
                                                              int(unit_seed)))

    def next_token_logits(self, max_length):
        """CausalLM::next_token_logits: a cached next-token function over the decode kernels."""
        return NextTokenLogits(self, max_length)

    def replay(self):
        N.host_check(N.host().pxa_lm_replay(self.h))

    def check_device_ids(self):
        """Raises PxkError (the reference's out-of-range message) if the last device-side pass saw
        an id outside [0, vocab)."""
        N.host_check(N.host().pxa_lm_check_device_ids(self.h))

    def last_logits_ptr(self):
        return N.host().pxa_lm_last_logits(self.h)

    def __del__(self):
        if getattr(self, "h", None):
            N.host().pxa_lm_destroy(self.h)
            self.h = None


class NextTokenLogits:
    """The function CausalLM::next_token_logits(max_length) returns: call it with the token ids so
    far to get the next token's logits (numpy, vocab floats). `callback` is the C function and
    context a Generate() binding takes."""

    def __init__(self, lm, max_length):
        self.lm = lm  # the function holds the model
        self.vocab = int(lm.cfg.vocab_size)
        self.h = N.host().pxa_lm_next_token_logits_create(lm.h, max_length)
        if not self.h:
            raise N.PxkError(N.host().pxa_last_error().decode())

    def __call__(self, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.int64)
        out = np.empty(self.vocab, np.float32)
        N.host_check(N.host().pxa_lm_next_token_logits(self.h, t.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)),
                                                       t.size, _p(out), self.vocab))
        return out

    @property
    def callback(self):
        """(function pointer, context) of pxa_lm_next_token_logits for this function."""
        return ctypes.cast(N.host().pxa_lm_next_token_logits, ctypes.c_void_p).value, self.h

    def __del__(self):
        if getattr(self, "h", None):
            N.host().pxa_lm_next_token_logits_destroy(self.h)
            self.h = None


def stream():
    return N.host().pxa_backend_stream()


def synchronize():
    N.host_check(N.host().pxa_backend_synchronize())


def launch_profile(run_once, reps=5):
    """Records every kernel launch of one call of run_once() on the backend (pxa_launch_log_*), then
    replays those launches in order `reps` times, each kernel recording its own start and end
    events. Returns one dict per launch: kernel (name and variant), family ("gemm", "attention",
    "rows"), algorithmic flops and bytes, seconds (the mean summed duration of its kernels) and the
    number of kernels it dispatched. The replays rewrite the outputs of the recorded pass."""
    h = N.host()
    N.host_check(h.pxa_launch_log_start())
    try:
        run_once()
    finally:
        count = ctypes.c_int64(0)
        N.host_check(h.pxa_launch_log_stop(ctypes.byref(count)))
    n = count.value
    secs = (ctypes.c_double * max(n, 1))()
    N.host_check(h.pxa_launch_log_time(reps, secs))
    out = []
    for i in range(n):
        kernel, family = ctypes.create_string_buffer(160), ctypes.create_string_buffer(32)
        flops, nbytes = ctypes.c_double(0), ctypes.c_double(0)
        N.host_check(h.pxa_launch_log_entry(i, kernel, 160, family, 32, ctypes.byref(flops), ctypes.byref(nbytes)))
        disp = ctypes.c_int32(0)
        N.host_check(h.pxa_launch_log_dispatches(i, ctypes.byref(disp)))
        out.append({"kernel": kernel.value.decode(), "family": family.value.decode(), "flops": flops.value,
                    "bytes": nbytes.value, "seconds": secs[i], "dispatches": disp.value})
    return out
