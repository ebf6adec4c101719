"""Graph replay for the torch.compile backend.

Every graph AOTAutograd hands the backend (training forward, backward, inference) is wrapped in a ReplayedGraph:
its first calls run op by op (warm-up: plan tuning happens there), the next one is captured once as a HIP graph
(omarchy_mac_torch.graphs.Graph: memory from graph pools, kept for the replays) and replayed, and every later call
is one graph launch. This is the step the reference names as its next lever for compiled graphs: static memory
planned once and the dispatch list recorded once (docs/roadmap.md:26-33; its stack plans replay a fixed dispatch
list, csrc/plans.cpp:280-294).

What a replay needs, and what it does when it does not have it:
  - Inputs. Parameters, buffers and the inputs a graph writes (AOTAutograd's metadata says which), and in the
    backward every tensor a replayed forward produced, are read in place by the graph. Any other input (the batch,
    the gradient of the loss) gets a buffer of its own, captured in its place, into which each call copies the new
    value. When an input read in place has moved (a parameter replaced), the forward is captured again at the new
    address, and if it moves again, with the input copied (an input the graph writes stays in place); after three
    captures the graph runs op by op. A backward whose saved tensors come from a forward that ran op by op runs op
    by op too.
  - Outputs. A replay rewrites the memory of the outputs of the previous one. The forward's outputs returned to the
    caller (the model's outputs) are copies. Tensors saved for the backward, new values of mutated inputs and the
    backward's gradients are new tensor objects over the graph's memory (autograd and the optimizer own them: a
    parameter's .grad is such a tensor until the next zero_grad). Before replaying, the graph checks that no tensor
    it handed out last time is still alive; if one is (a second forward before the previous backward, gradients
    accumulated over several backward passes without zero_grad(set_to_none=True)), the call runs op by op, which is
    always correct.
  - Capture. Inside a capture of the caller's own (a user-captured step, omarchy_mac_torch.graphs), a graph with
    host synchronization, CPU inputs or symbolic sizes, the call runs op by op. Dynamo makes sizes symbolic after a
    size changes; torch.compile(..., dynamic=False) keeps one graph per size instead, each replayed.

OMARCHY_MAC_TORCH_COMPILE_GRAPHS=0 (or set_enabled(False)) keeps every compiled graph op by op. STATS counts
captures, replays and op-by-op calls with their reasons.
"""

import os
import weakref

import torch

from omarchy_mac_torch import graphs
from omarchy_mac_torch.native import DEVICE, core

WARMUP_CALLS = 2
MAX_CAPTURES = 3
_enabled = os.environ.get("OMARCHY_MAC_TORCH_COMPILE_GRAPHS", "1") != "0"
# data pointers of storages that stay put while a captured graph lives (its inputs read in place, its input buffers,
# its outputs), each with its number of holders: a backward whose inputs are among them reads them in place. A graph
# holds its own memory (input buffers, outputs) until it is captured again; an input it reads in place is the
# caller's, held only while that storage lives (a finalizer drops it when the memory is freed, so that a later
# tensor at the same address is not taken for it)
_static_ptrs = {}


def _hold(p):
    _static_ptrs[p] = _static_ptrs.get(p, 0) + 1


def _drop(p):
    n = _static_ptrs.get(p, 0) - 1
    if n > 0:
        _static_ptrs[p] = n
    else:
        _static_ptrs.pop(p, None)


class _Holds:
    """A captured graph's entries in _static_ptrs: its own memory, and the caller's storages it reads in place (each
    dropped by a finalizer when that storage is freed). release() ends them all, once: when the graph is captured
    again or garbage-collected."""

    def __init__(self, owned, external):
        self.owned = owned
        self.external = {}
        for p in owned:
            _hold(p)
        for p, t in external:
            if p not in owned and p not in self.external:
                _hold(p)
                self.external[p] = weakref.finalize(t.untyped_storage(), _drop, p)

    def release(self):
        for p in self.owned:
            _drop(p)
        for p, fin in self.external.items():
            if fin.detach() is not None:  # the storage still lives: this graph's hold ends here
                _drop(p)
        self.owned, self.external = set(), {}
STATS = {"captures": 0, "replays": 0, "eager": 0, "reasons": {}}


def set_enabled(on):
    """Turns graph replay of compiled graphs on or off (graphs already captured stop replaying when off); returns the
    previous setting."""
    global _enabled
    prev, _enabled = _enabled, bool(on)
    return prev


def reset_stats():
    STATS.update(captures=0, replays=0, eager=0, reasons={})


def _ptr(t):
    return t.untyped_storage().data_ptr()


def _buffer_like(t):
    """A tensor of t's geometry holding t's value: captured in the place of an input that moves between calls."""
    return torch.empty_strided(t.size(), t.stride(), dtype=t.dtype, device=t.device).copy_(t)


class ReplayedGraph:
    """A compiled graph module's callable (boxed: called with the list of inputs), replayed as a HIP graph after
    WARMUP_CALLS op-by-op calls. kind: "forward", "backward" or "inference". For a forward or inference graph, outputs
    [user_from, user_to) are what the caller receives (copied after each replay); the others are handed out as
    tensors over the graph's memory."""

    def __init__(self, fn, kind, user_from=0, user_to=0, static_inputs=None, mutated_inputs=()):
        # an instance attribute: AOTAutograd wraps the backward's callable (torch._dynamo.disable), and the wrapper
        # takes over the instance's __dict__, where it looks for the flag
        self._boxed_call = True
        self.fn, self.kind = fn, kind
        self.user_span = (user_from, user_to) if kind != "backward" else (0, 0)
        self.calls = 0
        self.captures = 0
        self.eager_only = None  # reason this graph always runs op by op
        self.static_inputs = None if static_inputs is None else set(static_inputs)  # parameters and buffers
        self.mutated = set(mutated_inputs)  # inputs the graph writes: always read in place
        self.moves = {}         # input -> times it was found moved at a replay
        self.seen = None        # per input: the data pointer of the warm-up calls (None where it changed)
        self.graph = None

    # ---- the call ----

    def __call__(self, *args):
        a = list(args[0]) if len(args) == 1 and isinstance(args[0], list) else list(args)  # boxed, or not
        if self.eager_only is not None or not _enabled:
            return self._eager(a, self.eager_only or "disabled")
        if torch.cuda.is_current_stream_capturing():
            return self._eager(a, "inside a capture of the caller's")
        if self.graph is not None:
            return self._replay(a)
        if not all(isinstance(t, torch.Tensor) and t.device.type == DEVICE for t in a):
            self.eager_only = "inputs that are not device tensors (CPU tensors, symbolic sizes)"
            return self._eager(a, self.eager_only)
        self.calls += 1
        ptrs = core.storage_ptrs(a)
        self.seen = ptrs if self.seen is None else [p if p == q else None for p, q in zip(ptrs, self.seen)]
        if self.calls <= WARMUP_CALLS:
            return self._eager(a, "warm-up")
        if self.kind == "backward" and not any(p in _static_ptrs for p in ptrs):
            if self.calls > WARMUP_CALLS + 2:  # its forward is not replayed: copying every saved tensor would not pay
                self.eager_only = "forward not replayed"
            return self._eager(a, "forward not replayed yet")
        return self._capture(a)

    def _eager(self, a, why):
        STATS["eager"] += 1
        STATS["reasons"][why] = STATS["reasons"].get(why, 0) + 1
        return self.fn(*a)

    # ---- capture ----

    def _in_place(self, i, p):
        """Whether input i (data pointer p) is read in place by the captured graph: in the backward, a tensor of a
        replayed graph; in a forward, an input the graph writes, or else a parameter or buffer (Dynamo's static
        inputs; without that list, an input whose address stayed put over the warm-up calls) that has not moved more
        than once."""
        if self.kind == "backward":
            return p in _static_ptrs
        if i in self.mutated:
            return True
        if self.moves.get(i, 0) >= 2:
            return False
        if self.static_inputs is not None:
            return i in self.static_inputs
        return self.seen[i] == p

    def _capture(self, a):
        """Captures the graph on a, then runs it once. The liveness baseline is taken here, after _setup has
        returned: every reference _setup's locals held is gone, so each reference counted from now on that is not
        this object's own is a use."""
        self.captures += 1
        if self.captures > MAX_CAPTURES:
            self.eager_only = "inputs keep moving"
            return self._eager(a, self.eager_only)
        why = self._setup(a)
        if why is not None:  # an op that cannot be captured (host synchronization): op by op from now on
            self.eager_only = why
            return self._eager(a, why)
        self.watch.mark()
        STATS["captures"] += 1
        return self._run(a)

    def _setup(self, a):
        ptrs = core.storage_ptrs(a)
        static = [self._in_place(i, p) for i, p in enumerate(ptrs)]
        inputs = [t if keep else _buffer_like(t) for t, keep in zip(a, static)]
        graph = graphs.Graph()
        try:
            with graph.capture():
                outs = self.fn(*inputs)
        except Exception as e:
            graph.release()
            return f"not capturable ({type(e).__name__})"
        outs = list(outs)
        self.user = range(self.user_span[0], min(self.user_span[1], len(outs)))
        in_ptrs = {_ptr(t) for t, keep in zip(inputs, static) if keep}
        self.captured_ptrs = core.storage_ptrs(inputs)
        self.expected = [p if keep else 0 for p, keep in zip(self.captured_ptrs, static)]  # checked at each replay
        self.dynamic = [i for i, keep in enumerate(static) if not keep]
        # only the input buffers are kept: a reference to an input read in place (a saved tensor the forward handed
        # out, a parameter) would count as a use of it, and the graph needs its address alone
        self.inputs = [None if keep else t for t, keep in zip(inputs, static)]
        self.static = static
        self.template = [None if isinstance(o, torch.Tensor) else o for o in outs]
        self.user_outs = [(j, outs[j]) for j in self.user if isinstance(outs[j], torch.Tensor)]
        handed = [j for j, o in enumerate(outs) if isinstance(o, torch.Tensor) and j not in self.user]
        self.handed_idx = handed
        self.handed = core.StaticTensors([outs[j] for j in handed])
        # liveness: what a replay rewrites and someone else may hold (not the inputs read in place)
        watch = [outs[j] for j in handed if _ptr(outs[j]) not in in_ptrs]
        watch += [t for t, keep in zip(inputs, static) if not keep]
        self.watch = core.StaticTensors(watch)
        if self.graph is not None:
            self._forget()
            self.graph.release()
        self.graph = graph
        self.holds = _Holds({_ptr(t) for t, keep in zip(inputs, static) if not keep} |
                            {_ptr(o) for o in outs if isinstance(o, torch.Tensor)},
                            [(_ptr(t), t) for t, keep in zip(inputs, static) if keep])
        self.holds_gc = weakref.finalize(self, self.holds.release)
        return None

    def _forget(self):
        self.holds_gc.detach()
        self.holds.release()

    # ---- replay ----

    def _replay(self, a):
        moved = core.moved_inputs(a, self.expected)
        if moved:
            if self.kind == "backward":
                # saved tensors of a forward that ran op by op: this call too; of a forward captured again: again
                if not all(_ptr(a[i]) in _static_ptrs for i in moved):
                    return self._eager(a, "inputs from an op-by-op forward")
            else:  # captured again at the new address, and from a second move on with the input copied
                for i in moved:
                    self.moves[i] = self.moves.get(i, 0) + 1
            return self._capture(a)
        if self.watch.in_use():
            return self._eager(a, "outputs of the last replay still in use")
        return self._run(a)

    def _run(self, a):
        for i in self.dynamic:
            if a[i].data_ptr() != self.inputs[i].data_ptr():
                self.inputs[i].copy_(a[i])
        self.graph.replay()
        STATS["replays"] += 1
        out = list(self.template)
        for j, t in zip(self.handed_idx, self.handed.aliases()):
            out[j] = t
        for j, t in self.user_outs:
            out[j] = t.clone()
        return out


def wrap(gm_fn, kind):
    """The backend's callable for a rewritten graph module: a ReplayedGraph, told by AOTAutograd's metadata which
    forward outputs go back to the caller (mutated inputs' new values, then the model's outputs: the first
    num_forward_returns outputs; the rest are saved for the backward)."""
    if kind == "backward":
        return ReplayedGraph(gm_fn, kind)
    ctx = torch._guards.TracingContext.try_get()
    meta = getattr(ctx, "fw_metadata", None) if ctx is not None else None
    if meta is None:
        return ReplayedGraph(gm_fn, kind, 0, 1 << 30)  # every output treated as the caller's (copied)
    mutated = [i for i, info in enumerate(meta.input_info) if info.mutates_data or info.mutates_metadata]
    return ReplayedGraph(gm_fn, kind, meta.num_mutated_inp_runtime_indices, meta.num_forward_returns,
                         static_inputs=meta.static_input_indices or None, mutated_inputs=mutated)
