"""Seeded inputs for the gated delta-net recurrence (src/gdn.rs:17-77):
unit-scale q and k per head (|q|, |k| about 1, as after the L2 norm of the
model), gates below zero (decay), beta in [0, 1).
"""
from __future__ import annotations

import numpy as np


def gdn_case(synth, n_tok, h_k, h_v, s, seed, state_scale=0.1):
    r = synth.Rng(seed)
    q = r.normal(n_tok * h_k * s).reshape(n_tok, h_k, s) / np.float32(np.sqrt(s))
    k = r.normal(n_tok * h_k * s).reshape(n_tok, h_k, s) / np.float32(np.sqrt(s))
    v = r.normal(n_tok * h_v * s).reshape(n_tok, h_v, s)
    gate = -np.abs(r.normal(n_tok * h_v, 0.0, 0.5)).reshape(n_tok, h_v)
    beta = r.uniform(n_tok * h_v).reshape(n_tok, h_v).astype(np.float32)
    st = r.normal(h_v * s * s, 0.0, state_scale).reshape(h_v, s, s)
    return q, k, v, gate, beta, st
