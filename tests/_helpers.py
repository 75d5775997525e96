"""Shared helpers for the GPU parity tests: run the oracle on exactly the
inputs the GPU saw, and compare to the parity bar (ids bit-exact under the
margin guard; outputs within rtol = atol = 1e-2, plus a tighter relative
bound where fp32 accumulation allows it)."""
import numpy as np
import torch

from oracle import moe_oracle as O


def f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().to("cpu", torch.float64).numpy()


FORMATS = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16",
           torch.float8_e4m3fn: "fp8", torch.float4_e2m1fn_x2: "mxfp4"}


def expert_mats(buf: torch.Tensor, e: int, E: int, h: int, I: int):
    """(gate, up, down) of expert e from a packed buffer on any device, as fp64
    numpy arrays (expert_views on the flat layout, src/expert_layout.cuh:50-71;
    bf16 and fp8 buffers are decoded by the oracle from their raw bytes)."""
    if buf.dtype in (torch.bfloat16, torch.float8_e4m3fn, torch.float4_e2m1fn_x2):
        lo = O.weight_layout(E, h, I, FORMATS[buf.dtype])
        blk = buf.view(torch.uint8)[e * lo["expert_stride"]:(e + 1) * lo["expert_stride"]]
        return O.expert_matrices(blk.cpu().numpy(), 0, E, h, I, FORMATS[buf.dtype])
    es = buf.element_size()
    off = O.layout_offsets(E, h, I, es)
    base = e * off["expert_stride"] // es
    n = I * h
    g = buf[base:base + n].view(I, h)
    u = buf[base + n:base + 2 * n].view(I, h)
    d = buf[base + 2 * n:base + 3 * n].view(h, I)
    return f64(g), f64(u), f64(d)


def oracle_token(x: torch.Tensor, gate_w: torch.Tensor, buf: torch.Tensor, E: int, h: int,
                 I: int, k: int, renorm: bool):
    """Oracle for one token, fetching only the selected experts."""
    xn = f64(x)
    gw = f64(gate_w)
    logits64 = O.router_logits(gw, xn)
    probs, ids, ws = O.softmax_topk(logits64.astype(np.float32), k, renorm)
    m = logits64.max()
    p64 = np.exp(logits64 - m)
    p64 /= p64.sum()
    w64 = p64[ids]
    if renorm:
        w64 = w64 / w64.sum()
    out = np.zeros(h)
    for kk in range(k):
        g, u, d = expert_mats(buf, int(ids[kk]), E, h, I)
        out += w64[kk] * O.expert_ffn(xn, g, u, d)
    robust = O.selection_is_robust(gw, xn, k)
    return {"out": out, "ids": ids, "weights": ws, "robust": robust}


def oracle_rows(x: torch.Tensor, gate_w: torch.Tensor, buf: torch.Tensor, E: int, h: int,
                I: int, k: int, renorm: bool):
    """oracle_token for every row of x [B, h], fetching each selected expert
    from the device once for all the rows that select it (the FFN of those
    rows as one fp64 matrix product: expert_ffn on an [h, n] block).  Returns
    one dict per row, as oracle_token."""
    xn = f64(x).reshape(-1, h)
    gw = f64(gate_w)
    rows, users = [], {}
    for b in range(xn.shape[0]):
        logits64 = O.router_logits(gw, xn[b])
        _, ids, ws = O.softmax_topk(logits64.astype(np.float32), k, renorm)
        p64 = np.exp(logits64 - logits64.max())
        p64 /= p64.sum()
        w64 = p64[ids]
        if renorm:
            w64 = w64 / w64.sum()
        rows.append({"out": np.zeros(h), "ids": ids, "weights": ws, "w64": w64,
                     "robust": O.selection_is_robust(gw, xn[b], k)})
        for kk in range(k):
            users.setdefault(int(ids[kk]), []).append((b, kk))
    for e, lst in sorted(users.items()):
        g, u, d = expert_mats(buf, e, E, h, I)
        y = O.expert_ffn(xn[[b for b, _ in lst]].T, g, u, d)  # [h, n]
        for j, (b, kk) in enumerate(lst):
            rows[b]["out"] += rows[b]["w64"][kk] * y[:, j]
        del g, u, d
    return rows


def assert_parity(got_out, got_ids, got_w, ref, rel_tol=1e-4, w_rtol=1e-5, label=""):
    """The parity bar: ids bit-exact (the case must pass the margin guard),
    weights within w_rtol, output within rtol = atol = 1e-2 and within
    rel_tol of max|ref| (max-abs error, tests/test_correctness.cu:121-130)."""
    assert ref["robust"], f"{label}: selection not robust to fp32 rounding; pick another seed"
    if got_ids is not None:
        np.testing.assert_array_equal(got_ids.cpu().numpy().reshape(-1), ref["ids"],
                                      err_msg=f"{label}: expert ids")
    if got_w is not None:
        np.testing.assert_allclose(got_w.cpu().numpy().reshape(-1), ref["weights"], rtol=w_rtol,
                                   atol=1e-7, err_msg=f"{label}: gate weights")
    g = f64(got_out).reshape(-1)
    np.testing.assert_allclose(g, ref["out"], rtol=1e-2, atol=1e-2, err_msg=f"{label}: output")
    err = O.relative_error(g, ref["out"])
    assert err < rel_tol, f"{label}: relative error {err:.3e} >= {rel_tol:.1e}"
    return err


def assert_same_up_to_order(got: torch.Tensor, want: torch.Tensor, label="", tol=None):
    """Two GPU paths that compute the same fp32 dot products in a different
    summation order: max|got - want| <= tol * max|want|, tol = 1e-5 for fp32
    outputs (a few ulps of reordering error) and 2e-3 for fp16 outputs (one
    fp16 rounding step, 2^-10 relative), unless given."""
    assert got.dtype == want.dtype and got.shape == want.shape, label
    if tol is None:
        tol = 2e-3 if got.dtype == torch.float16 else 1e-5
    g, w = f64(got), f64(want)
    err = np.abs(g - w).max() if g.size else 0.0
    assert err <= tol * max(np.abs(w).max(), 1e-30), f"{label}: max diff {err:.3g}"
