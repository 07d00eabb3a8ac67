"""Per-layer capture of the tagged persistent kernel and the strict per-layer
check against the oracle, shared by the full-depth GPU tests.

With ``fusion_groups = num_layers`` every layer is its own persistent launch,
and after each launch the workspace's tagged exchange holds that layer's
intermediates (qkv, attention output, o_proj, SiLU*mul, down) and the residual
after the post-attention add (published at every segment end but the last).
The oracle is then fed, layer by layer, the kernel's OWN input to that layer,
so every comparison is between identical inputs: each GEMV and attention
output must be within one bf16 ulp at its row's scale (SiLU*mul within that
error carried through its product, ``act_excess``), and the logits (the oracle's last layer
and head on the kernel's last-layer input) within 2e-2. Rounding flips cannot
compound over depth in this check, so no depth allowance is needed."""

from __future__ import annotations

import torch

from gpu_support import VOCAB, max_abs

LOGIT_TOL = 2e-2
ULP_TOL = 1.0
# tagged region -> (width per row, oracle trace key)
REGIONS = {"tw_qkv": (4096, "qkv"), "tw_attn": (2048, "attn"), "tw_o": (1024, "o"),
           "tw_act": (3072, "act"), "tw_down": (1024, "down"), "tw_res2": (1024, "resid_post")}


def ulp_row_scale(ref: torch.Tensor) -> torch.Tensor:
    """One bf16 ulp at each row's max magnitude (per-row tolerance unit)."""
    m = ref.abs().amax(dim=-1, keepdim=True).clamp_min(1e-30)
    return torch.pow(2.0, torch.floor(torch.log2(m)) - 7)


def ulp_excess(got: torch.Tensor, ref: torch.Tensor) -> float:
    return ((got.float() - ref.float()).abs() / ulp_row_scale(ref.float())).max().item()


def act_excess(got: torch.Tensor, gate: torch.Tensor, up: torch.Tensor, ref: torch.Tensor) -> float:
    """SiLU(g)*u is not a GEMV output: it multiplies two of them, each within
    one ulp at its row's scale. Its bound is that error carried through the
    product, |silu'(g) u| ulp(g) + |silu(g)| ulp(u), plus one ulp of the element
    for the two roundings (kernel and oracle). Returns the largest |diff| in
    units of that bound (<= 1 passes)."""
    g, u = gate.float(), up.float()
    sig = torch.sigmoid(g)
    dsilu = sig * (1 + g * (1 - sig))
    prop = (dsilu * u).abs() * ulp_row_scale(g) + (g * sig).abs() * ulp_row_scale(u)
    r = ref.float()
    elem_ulp = torch.pow(2.0, torch.floor(torch.log2(r.abs().clamp_min(1e-30))) - 7)
    return ((got.float() - r).abs() / (prop + elem_ulp)).max().item()


class LayerCapture:
    """``on_segment`` callback for ``TaskGraphDecoder.decode_rows``: after each
    one-layer launch, decode the tagged regions of replica 0 for ``rows`` rows."""

    def __init__(self, dec, rows: int):
        from nanovllm.backends.megakernel import native

        self.dec, self.rows = dec, rows
        self.layout = native.workspace_layout()
        self.native = native
        self.layers: list[dict[str, torch.Tensor]] = []

    def __call__(self, index: int, segment) -> None:
        layers = sorted({t.layer for row in segment.rows for t in row if t.op == self.native.OP_QKV})
        assert layers == [index], f"segment {index} holds layers {layers}; expected one layer per launch"
        ws = self.dec._workspace
        out = {}
        for name, (width, key) in REGIONS.items():
            off, size = self.layout[name]
            vals, tags = self.native.decode_tagged_bf16(ws[off:off + size].cpu(), self.rows, width)
            fresh = bool(((tags & 31) == index).all()) and tags.unique().numel() == 1
            if name == "tw_res2" and not fresh:
                continue  # the last launch does not publish the residual
            assert fresh, f"layer {index}: {name} words not all written by this layer ({tags.unique().tolist()[:4]})"
            out[key] = vals.to(torch.bfloat16)
        self.layers.append(out)


def per_layer_check(oracle, capture: LayerCapture, ids, positions, tables, k_cache, v_cache, logits,
                    tokens, label: str = "") -> dict:
    """Feed the oracle the kernel's input to every layer and compare. Returns a
    summary (worst ulp per intermediate, logit error, token agreement)."""

    rows = len(ids)
    worst = {key: 0.0 for _, key in REGIONS.values()}
    hidden, residual = oracle.embed_rows(ids), None
    n = len(capture.layers)
    assert n == oracle.num_layers, f"captured {n} layers of {oracle.num_layers}"
    for l, kern in enumerate(capture.layers):
        trace = {}
        o_hidden, o_res = oracle.layer(l, hidden, residual, positions, tables, k_cache, v_cache, trace=trace)
        for key, got in kern.items():
            if key == "act":
                ex = act_excess(got[:rows], trace["gate"], trace["up"], trace["act"])
            else:
                ex = ulp_excess(got[:rows], trace[key])
            worst[key] = max(worst[key], ex)
            assert ex <= ULP_TOL + 1e-6, f"{label} layer {l} {key}: {ex:.2f} ulp at row scale"
        if l + 1 < n:
            assert "resid_post" in kern, f"layer {l}: residual not published"
            hidden, residual = kern["down"][:rows], kern["resid_post"][:rows]
        else:
            hidden, residual = o_hidden, o_res
    ref_logits, ref_toks = oracle.head(hidden, residual)
    ref_logits = ref_logits.float()
    err = max_abs(logits, ref_logits)
    assert err <= LOGIT_TOL, f"{label} logits max |diff| {err:.3e} > {LOGIT_TOL}"
    for b, (t, r) in enumerate(zip(tokens, ref_toks)):
        # the argmax itself is exact: the kernel's token is the first maximal index of its own logits
        assert t == int(torch.argmax(logits[b])), f"{label} row {b}: token {t} is not the argmax of its logits"
        if t != r:
            gap = (ref_logits[b, r] - ref_logits[b, t]).item()
            assert gap <= LOGIT_TOL, f"{label} row {b}: token {t} vs oracle {r}, oracle gap {gap:.3e}"
    return {"worst_ulp": worst, "max_dlogit": err, "tokens": tokens, "oracle_tokens": ref_toks}


def step_logits_buffer(rows: int) -> torch.Tensor:
    return torch.zeros(rows, VOCAB, dtype=torch.bfloat16, device="cuda")
