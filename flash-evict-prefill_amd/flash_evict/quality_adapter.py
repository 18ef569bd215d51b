"""Several eviction policies from one shared prefill, decoded as one batch (reference
flash_evict/quality_adapter.py:19-136 in anishesg/flash-evict-prefill).

`PairedController(model)` runs the prompt forward once for a group of policies that need the
same attention output and scores (`group_key`), and stores each policy's compacted K/V in
`bank[name][layer]`. `activate(names)` stacks the named caches along the batch for
`decode_batch`, greedy decoding of all of them together. A policy is a dict with `name`,
`backend` ("full", "snap", "fused", "value_norm_only", "uniform_recent") and `budget`;
fused policies also carry recency_decay, observation_window, value_weighted and
reserved_recent.
"""
import torch

from .baselines import flash_attention, snap_scores, snap_select
from .cache import gather_tokens
from .controller import SNAP_WINDOW, Controller
from .prefill import prefill, select_tokens

__all__ = ["PairedController", "choose_indices", "decode_batch", "default_methods", "group_key"]

_FUSED_SCORING = ("recency_decay", "observation_window", "value_weighted")


def default_methods():
    """The evaluation's policy list: the full cache, SnapKV and three fused policies at
    budgets 256 and 1024, and two 256-token ablations (quality_adapter.py:19-31)."""
    methods = [dict(name="full", backend="full", budget=None)]
    for budget in (256, 1024):
        methods.append(dict(name="snap_%d" % budget, backend="snap", budget=budget))
        for label, window, recent in (("d01_r0", 0, 0), ("d0.1_w128_r0", 128, 0), ("d0.1_w128_r64", 128, 64)):
            methods.append(dict(name="%s_%d" % (label, budget), backend="fused", budget=budget, recency_decay=.1,
                                observation_window=window, value_weighted=True, reserved_recent=recent))
    methods += [dict(name="%s_256" % backend, backend=backend, budget=256)
                for backend in ("value_norm_only", "uniform_recent")]
    return methods


def group_key(method):
    """Policies that can share one prefill have equal keys: every baseline uses the same
    attention output; fused policies need equal scoring (quality_adapter.py:34-37)."""
    if method["backend"] != "fused":
        return ("baseline",)
    return ("fused",) + tuple(method[key] for key in _FUSED_SCORING)


# Selectors: (k, v, budget, method, importance, snap) -> kept indices [B, Hkv, budget].
def _keep_suffix(k, v, budget, method, importance, snap):
    # the newest `budget` tokens, no attention sink reserved
    n = k.shape[2]
    return torch.arange(n - budget, n, device=k.device).expand(k.shape[0], k.shape[1], budget)


def _keep_largest_values(k, v, budget, method, importance, snap):
    return select_tokens(v.float().abs().sum(-1), budget)[0]


def _keep_snap(k, v, budget, method, importance, snap):
    return snap_select(snap, budget, window=SNAP_WINDOW, kernel=5)[0]


def _keep_fused(k, v, budget, method, importance, snap):
    return select_tokens(importance, budget, reserved_recent=min(budget, method["reserved_recent"]))[0]


_SELECTORS = {"uniform_recent": _keep_suffix, "value_norm_only": _keep_largest_values, "snap": _keep_snap,
              "fused": _keep_fused}


def choose_indices(method, k, v, importance=None, snap=None):
    """Kept indices of one policy, or None when it keeps every token (the full cache, or a
    budget covering the prompt)."""
    n = k.shape[2]
    budget = n if method["budget"] is None else min(n, method["budget"])
    if method["backend"] == "full" or budget >= n:
        return None
    try:
        selector = _SELECTORS[method["backend"]]
    except KeyError:
        raise ValueError("Unknown policy backend %r" % (method["backend"],)) from None
    return selector(k, v, budget, method, importance, snap)


class PairedController(Controller):
    def __init__(self, model):
        super().__init__(model)
        self.bank = {}
        self.active_methods = []

    def prepare(self, methods, length=None):
        """Start a shared prefill for `methods` (one `group_key`) of a `length`-token prompt."""
        methods = list(methods)
        if not methods or len({group_key(m) for m in methods}) != 1:
            raise ValueError("A shared prefill requires identical attention output and score settings")
        self.reset()
        self.position_end = length
        self.active_methods = methods
        self.bank = {m["name"]: {} for m in methods}

    def _prefill_layer(self, layer, q, k, v, scaling):
        lead = self.active_methods[0]
        n = k.shape[2]
        importance = snap = None
        if lead["backend"] == "fused":
            out, importance = prefill(q, k, v, scale=scaling, **{key: lead[key] for key in _FUSED_SCORING})
        else:
            out = flash_attention(q, k, v)
            if any(m["backend"] == "snap" and m["budget"] < n for m in self.active_methods):
                snap = snap_scores(q, k, SNAP_WINDOW)
        for m in self.active_methods:
            keep = choose_indices(m, k, v, importance, snap)
            self.bank[m["name"]][layer] = (
                {"k": k, "v": v} if keep is None else {"k": gather_tokens(k, keep), "v": gather_tokens(v, keep)})
        return out

    def activate(self, names, *, consume=True):
        """Stack the named policies' caches along the batch as the decode cache. They must
        retain the same number of tokens; with `consume` they leave the bank."""
        caches = [self.bank[name] for name in names]
        kept = {c[layer]["k"].shape[2] for c in caches for layer in c}
        if len(kept) != 1:
            raise ValueError("Batched policies must retain the same number of tokens, got %s" % sorted(kept))
        stacked = {}
        for layer in caches[0]:
            parts = {key: [c[layer][key] for c in caches] for key in ("k", "v")}
            stacked[layer] = {key: (t[0] if len(t) == 1 else torch.cat(t, 0)) for key, t in parts.items()}
        self.states = stacked
        self.mode = "decode"
        self.method = "full"
        if consume:
            for name in names:
                self.bank.pop(name)


@torch.inference_mode()
def decode_batch(model, ctl, last_token, prompt_length, max_new_tokens, stop_ids, *, suppress_first_stop=False):
    """Greedy decoding of every cache stacked by `ctl.activate(...)`, starting from the
    prompt's last token at position prompt_length-1. Returns, per batch row, the generated
    ids up to and including its first stop id (quality_adapter.py:115-136)."""
    batch = next(iter(ctl.states.values()))["k"].shape[0]
    device = next(model.parameters()).device
    stops = torch.tensor(sorted(stop_ids), dtype=torch.long, device=device)
    token = torch.full((batch, 1), int(last_token), dtype=torch.long, device=device)
    produced = torch.zeros((batch, max_new_tokens), dtype=torch.long, device=device)
    length = torch.full((batch,), max_new_tokens, dtype=torch.long, device=device)
    running = torch.ones(batch, dtype=torch.bool, device=device)
    for step in range(max_new_tokens):
        position = prompt_length - 1 + step
        ctl.position_end = position + 1
        pos = torch.full((batch, 1), position, dtype=torch.long, device=device)
        logits = model.lm_head(model.model(token, position_ids=pos, use_cache=False).last_hidden_state[:, -1])
        if suppress_first_stop and step == 0 and stops.numel():
            logits[:, stops] = -torch.inf
        token = logits.argmax(-1, keepdim=True)
        produced[:, step] = token[:, 0]
        stopped = running & torch.isin(token[:, 0], stops)
        length = torch.where(stopped, torch.full_like(length, step + 1), length)
        running &= ~stopped
        if not bool(running.any()):
            break
    rows = produced.cpu().tolist()
    return [row[:n] for row, n in zip(rows, length.cpu().tolist())]
