"""Oracle: per-row entropy, gate, penalty, argmax / top-K and top-p sampling
(test infrastructure only).

Restates
  * compute_entropy (core/generator_utils.py:196-202): H = -sum softmax(x/T) *
    log_softmax(x/T), NaN terms dropped; here in float64.
  * apply_repetition_penalty (core/generator_utils.py:205-230): on the unique
    generated ids, x > 0 ? x / p : x * p computed in float32 (torch's CPU
    scalar division and multiplication are single IEEE operations in the
    tensor's dtype) and rounded to the logits dtype.
  * _do_extend / _do_branch keys (core/generator.py:283-287, :308-310): the
    log_softmax of the penalised logits as torch forms it,
    fl(fl(x - max) - log(sum exp(x - max))) rounded to the logits dtype;
    argmax = first index of the maximum; top-K = K largest, ties to the
    lowest index (fixed here; torch.topk leaves it unspecified).
  * adaptive_threshold (core/generator_utils.py:247-253) and the gate of
    _step_leaf (core/generator.py:333-374).
  * the bit-exact temperature + top-p sampler specified in csrc/sampling_ref.c,
    through ctypes on oracle/_build/liboracle.so.

Pinned by (tests/test_oracle_sampling.py): Philox4x32-10 known answers
(Random123's published vectors, reproduced by rocRAND's independent engine,
tests/golden/philox_rocrand.json); det_exp2 exact on integers and within
1e-6 of 2^y; entropy closed forms (uniform -> ln V, one dominant logit -> 0)
and agreement with torch's own log_softmax / topk on random rows; the
nucleus of the fixed-point rule equals HuggingFace TopP's float64 rule on
random rows away from the boundary; a chi-square test of the draws against
the renormalised nucleus distribution.
"""
from __future__ import annotations

import ctypes
import math
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(HERE, "_build", "liboracle.so")
        if not os.path.exists(path):
            from .build import build

            build()
        L = ctypes.CDLL(path)
        L.oracle_philox4x32_10.argtypes = [ctypes.POINTER(ctypes.c_uint32)] * 3
        L.oracle_philox4x32_10.restype = None
        L.oracle_det_exp2.argtypes = [ctypes.c_float]
        L.oracle_det_exp2.restype = ctypes.c_float
        L.oracle_det_q.argtypes = [ctypes.c_float]
        L.oracle_det_q.restype = ctypes.c_uint64
        L.oracle_top_p_sample.argtypes = [
            ctypes.POINTER(ctypes.c_float), ctypes.c_int32, ctypes.c_float, ctypes.c_float,
            ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint32,
            ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64),
        ]
        L.oracle_top_p_sample.restype = ctypes.c_int32
        _LIB = L
    return _LIB


def philox4x32_10(counter, key):
    c = (ctypes.c_uint32 * 4)(*[int(x) & 0xFFFFFFFF for x in counter])
    k = (ctypes.c_uint32 * 2)(*[int(x) & 0xFFFFFFFF for x in key])
    o = (ctypes.c_uint32 * 4)()
    lib().oracle_philox4x32_10(c, k, o)
    return list(o)


def det_exp2(y: float) -> float:
    return lib().oracle_det_exp2(float(y))


def det_q(y: float) -> int:
    return lib().oracle_det_q(float(y))


def sample_scale(temperature: float) -> np.float32:
    """c = fp32(log2(e) / T), the factor the sampler applies (kernel: samp_c)."""
    return np.float32(1.4426950408889634 / float(temperature))


def top_p_sample(xp: np.ndarray, temperature: float, top_p: float, seed: int, step: int, row: int):
    """Draw per csrc/sampling_ref.c. Returns (index, kept, Z, need)."""
    x = np.ascontiguousarray(xp, dtype=np.float32)
    kept = ctypes.c_int32()
    z = ctypes.c_uint64()
    need = ctypes.c_uint64()
    idx = lib().oracle_top_p_sample(
        x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), x.size, sample_scale(temperature),
        np.float32(top_p), seed, step, row, ctypes.byref(kept), ctypes.byref(z), ctypes.byref(need))
    return int(idx), kept.value, z.value, need.value


# ---- dtype rounding --------------------------------------------------------------------------
def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float32 values to bf16 / f16 (nearest even) and back; identity for f32."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "f32":
        return x
    if dtype == "f16":
        return x.astype(np.float16).astype(np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    r = np.where(nan, u | 0x400000, r)
    return r.astype(np.uint32).view(np.float32)


def penalize(x: np.ndarray, ids, penalty: float, dtype: str) -> np.ndarray:
    """apply_repetition_penalty (core/generator_utils.py:205-230) on float32 values."""
    x = np.asarray(x, dtype=np.float32).copy()
    if not len(ids) or penalty == 1.0:
        return x
    u = np.unique(np.asarray(ids, dtype=np.int64))
    g = x[u]
    p = np.float32(penalty)
    x[u] = round_to(np.where(g > 0, g / p, g * p).astype(np.float32), dtype)
    return x


def entropy(x: np.ndarray, temperature: float = 1.0) -> float:
    """compute_entropy in float64 (nats)."""
    z = np.asarray(x, dtype=np.float64) / float(temperature)
    z = z - z.max()
    lse = math.log(np.exp(z).sum())
    lp = z - lse
    p = np.exp(lp)
    t = p * lp
    t = np.where(np.isnan(t), 0.0, t)
    return float(-t.sum())


LOG2E_F32 = np.float32(1.4426950408889634)


def _softmax_state(y: np.ndarray):
    """(m, fl(y - m), s, ln s) of a row of dtype values, as torch's device softmax and
    log_softmax form them: e = exp2(fl(y - m) * fl(log2 e)), s = sum e (here exact in
    float64, rounded to float once; torch sums in float in its own order)."""
    m = np.float32(y.max())
    d = (y - m).astype(np.float32)
    e = np.exp2(d * LOG2E_F32).astype(np.float32)
    s = np.float32(e.astype(np.float64).sum())
    return m, d, e, s, np.float32(np.log(s))


def entropy_chain(x: np.ndarray, temperature: float, dtype: str) -> float:
    """compute_entropy (core/generator_utils.py:196-202) with the rounding torch's
    device kernels give it in the logits dtype (the reference calls it on bf16
    logits for a bf16 model, core/generator.py:342, :293):
      y = rnd(x * fl(1/T))            (a tensor divided by a Python float is
                                        multiplied by the float reciprocal)
      p = rnd(e / s), lp = rnd(fl(y - m) - ln s)   (softmax, log_softmax)
      t = rnd(p * lp), NaN -> 0       (probs * log_probs, nan_to_num)
      H = -rnd(sum t)                 (the sum exact in float64, rounded once)
    rnd rounds to `dtype` (identity for f32). Returns H as a Python float."""
    x = np.asarray(x, dtype=np.float32)
    inv = np.float32(1.0) / np.float32(temperature)
    y = round_to(x * inv, dtype)
    _, d, e, s, logs = _softmax_state(y)
    with np.errstate(invalid="ignore", divide="ignore"):
        p = round_to((e / s).astype(np.float32), dtype)
        lp = round_to((d - logs).astype(np.float32), dtype)
        t = round_to((p * lp).astype(np.float32), dtype)
    t = np.where(np.isnan(t), np.float32(0.0), t)
    S = np.float32(t.astype(np.float64).sum())
    return float(-round_to(np.array([S], dtype=np.float32), dtype)[0])


def log_softmax_keys(xp: np.ndarray, dtype: str) -> np.ndarray:
    """log_softmax as torch's device kernel forms it, rounded to the logits dtype
    (float32 values): rnd(fl(x - m) - ln s), s from _softmax_state."""
    xp = np.asarray(xp, dtype=np.float32)
    _, d, _, _, logs = _softmax_state(xp)
    return round_to((d - logs).astype(np.float32), dtype)


def topk(keys: np.ndarray, k: int):
    """K largest keys, ties to the lowest index. Returns (ids, values)."""
    order = np.lexsort((np.arange(keys.size), -keys.astype(np.float64)))[:k]
    return order.astype(np.int64), keys[order]


def adaptive_threshold(base_val: float, max_active: int, current_active: int) -> float:
    """core/generator_utils.py:247-253."""
    util = current_active / max(max_active, 1)
    return base_val * (1.0 + 2.0 * util * util)


def soft_explore_factor(step: int, window: int, initial: float) -> float:
    """core/generator.py:319-331."""
    if step >= window:
        return 1.0
    t = step / max(window, 1)
    return initial + (1.0 - initial) * t


def hf_top_p_keep(x: np.ndarray, temperature: float, top_p: float) -> np.ndarray:
    """HuggingFace TemperatureLogitsWarper + TopPLogitsWarper kept-set in float64
    (transformers generation/logits_process.py:301-303, :527-540): sort ascending,
    remove where cumsum(softmax) <= 1 - top_p, keep at least the largest."""
    z = np.asarray(x, dtype=np.float64) / float(temperature)
    order = np.argsort(z, kind="stable")
    p = np.exp(z[order] - z.max())
    p /= p.sum()
    cum = np.cumsum(p)
    remove = cum <= 1.0 - top_p
    remove[-1] = False
    keep = np.zeros(x.size, dtype=bool)
    keep[order[~remove]] = True
    return keep


def reference_cpu_rows(logits, temperature: float, top_p: float, gate_threshold: float, seed: int = 0):
    """The reference's per-row CPU path in torch, in the logits dtype: the
    entropy gate of _step_leaf (compute_entropy at the gate temperature,
    core/generator_utils.py:196-202, core/generator.py:342) and HF sampling
    (TemperatureLogitsWarper + TopPLogitsWarper + multinomial,
    transformers generation/logits_process.py:301-303, :527-540,
    generation/utils.py:2923), one row at a time as the generator does.
    Used as the timed CPU baseline. Returns (entropies, gate flags, ids)."""
    import torch

    g = torch.Generator().manual_seed(seed)
    ents, gates, ids = [], [], []
    for x in logits:
        z = x / temperature
        p = torch.softmax(z, dim=-1)
        lp = torch.log_softmax(z, dim=-1)
        t = p * lp
        h = -torch.where(torch.isnan(t), torch.zeros_like(t), t).sum().item()
        ents.append(h)
        gates.append(h > gate_threshold)
        s, order = torch.sort(z, descending=False)
        cum = s.softmax(dim=-1).cumsum(dim=-1)
        remove = cum <= (1 - top_p)
        remove[-1:] = False
        z2 = z.clone()
        z2[order[remove]] = -float("inf")
        ids.append(int(torch.multinomial(torch.softmax(z2.float(), dim=-1), 1, generator=g)))
    return ents, gates, ids
