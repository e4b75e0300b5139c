"""Shared helpers for the GPU parity tests: run a workload through the HIP
library (via its C-ABI) and through the CPU oracle, and compare."""
from __future__ import annotations

import os

import numpy as np

BOUNDARY = 1e-6      # |u - CDF boundary| or |nucleus cumulative - p| below this is ambiguous
MINP_BOUNDARY = 1e-12  # |exp(l) - threshold| / threshold at the min-p cut below this is ambiguous
PROB_RTOL = 1e-5     # post-filter probability tolerance (relative)


def to_device(w, device="cuda"):
    import torch

    if w.logits.dtype == np.uint16:
        logits = torch.from_numpy(w.logits.view(np.int16)).view(torch.bfloat16).to(device)
    else:
        logits = torch.from_numpy(w.logits).to(device)
    off = ids = None
    if w.hist_offsets is not None:
        off = torch.from_numpy(w.hist_offsets.astype(np.int64)).to(device)
        ids = torch.from_numpy(w.hist_ids.astype(np.uint32).view(np.int32)).to(device)
    return logits, off, ids


def run_gpu(w, logits=None, off=None, ids=None):
    import torch

    from lmrs_amd import sampling as S

    if logits is None:
        logits, off, ids = to_device(w)
    res = S.sample_batch(logits, hist_offsets=off, hist_ids=ids, repetition_penalty=w.repetition_penalty,
                         presence_penalty=w.presence_penalty, frequency_penalty=w.frequency_penalty,
                         temperature=w.temperature, top_k=w.top_k, top_p=w.top_p, uniforms=w.uniforms,
                         min_p=w.min_p, dist=True)
    torch.cuda.synchronize()
    return {
        "token_id": res["token_ids"].cpu().numpy().view(np.uint32),
        "log_prob": res["log_probs"].cpu().numpy(),
        "logit": res["logits"].cpu().numpy(),
        "status": res["status"].cpu().numpy(),
        "kept_count": res["kept_count"].cpu().numpy(),
        "kept_mass": res["kept_mass"].cpu().numpy(),
    }


def run_oracle(w, threads=None):
    import oracle as O

    params = [O.make_params(float(w.repetition_penalty[r]), float(w.presence_penalty[r]),
                            float(w.frequency_penalty[r]), float(w.temperature[r]), int(w.top_k[r]),
                            float(w.top_p[r]), -1.0 if w.min_p is None else float(w.min_p[r]))
              for r in range(w.batch)]
    threads = threads or min(16, os.cpu_count() or 1)
    return O.sample_batch(w.logits, w.hist_offsets, w.hist_ids, params, w.uniforms, n_threads=threads)


def compare(gpu, ref):
    """Returns a report dict; asserts nothing."""
    st_gpu = gpu["status"] & 0xFF
    ok = ref["status"] == 0
    boundary = ok & ((ref["cdf_margin"] < BOUNDARY) | (ref["top_p_margin"] < BOUNDARY)
                     | (ref["min_p_margin"] < MINP_BOUNDARY))
    same = gpu["token_id"] == ref["token_id"]
    status_mismatch = int(np.sum(st_gpu != ref["status"]))
    mism = ok & ~same & ~boundary
    both = ok & same
    prob_gpu = np.exp(gpu["log_prob"].astype(np.float64))
    rel = np.abs(prob_gpu - ref["prob"]) / np.maximum(ref["prob"], 1e-300)
    # near a boundary the kept set itself is ambiguous (a nucleus cumulative
    # within 1e-6 of top_p may keep one token more or fewer), and with it the
    # normaliser: those rows are counted, not held to the probability bar
    rel = np.where(both & ~boundary, rel, 0.0)
    logit_bad = int(np.sum(both & (gpu["logit"].view(np.uint32) != ref["logit"].view(np.uint32))))
    # The GPU's near-boundary flag against the oracle's margins: rows well
    # inside the margin must carry it, rows well outside must not (the two
    # compute their sums in different orders, so a band around the margin
    # itself is left to either side).  Rows with a min-p cut are only checked
    # one way: the GPU tests the keys on both sides of the cut whether or not
    # an element holds them, so it may flag a row whose elements all lie
    # clear of the threshold.
    flag = (gpu["status"] & 0x100) != 0
    mg = np.minimum(ref["cdf_margin"], ref["top_p_margin"])
    must = ok & ((mg < 0.5 * BOUNDARY) | (ref["min_p_margin"] < 0.5 * MINP_BOUNDARY))
    must_not = ok & (mg > 2 * BOUNDARY) & np.isinf(ref["min_p_margin"])
    # the post-filter distribution (kept count and mass, when the GPU reports
    # them): every kept token's probability is exp(l - max) / mass over the
    # first `count` of the sorted order, so these two pin all of them
    dist = {}
    if "kept_count" in gpu:
        clean = ok & ~boundary
        kc, km = gpu["kept_count"], gpu["kept_mass"]
        counted = clean & (kc >= 0)
        mrel = np.abs(km - ref["sum_kept"]) / np.maximum(np.abs(ref["sum_kept"]), 1e-300)
        dist = {"kept_count_mismatch": int(np.sum(counted & (kc != ref["n_kept"]))),
                "kept_count_unreported": int(np.sum(clean & (kc < 0))),
                "kept_mass_max_rel_err": float(np.max(np.where(clean, mrel, 0.0))) if len(ok) else 0.0}
    return {
        **dist,
        "rows": int(len(ok)),
        "status_mismatch": status_mismatch,
        "token_mismatch": int(np.sum(mism)),
        "boundary_rows": int(np.sum(boundary)),
        "boundary_mismatch": int(np.sum(boundary & ~same)),
        "gpu_flagged": int(np.sum((gpu["status"] & 0x100) != 0)),
        "max_prob_rel_err": float(np.max(rel)) if len(rel) else 0.0,
        "logit_mismatch": logit_bad,
        "flag_missing": int(np.sum(must & ~flag)),
        "flag_extra": int(np.sum(must_not & flag)),
        "mismatch_rows": np.nonzero(mism)[0][:10].tolist(),
    }


def assert_parity(rep, name=""):
    assert rep["status_mismatch"] == 0, (name, rep)
    assert rep["token_mismatch"] == 0, (name, rep)
    assert rep["logit_mismatch"] == 0, (name, rep)
    assert rep["max_prob_rel_err"] < PROB_RTOL, (name, rep)
    assert rep["flag_missing"] == 0 and rep["flag_extra"] == 0, (name, rep)
    if "kept_count_mismatch" in rep:
        assert rep["kept_count_mismatch"] == 0, (name, rep)
        assert rep["kept_mass_max_rel_err"] < PROB_RTOL, (name, rep)
