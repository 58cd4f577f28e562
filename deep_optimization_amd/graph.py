"""Whole-step HIP graph capture of a (compressed) model's training step.

Mirrors Activation_Compression/cuda_graph_utils.py: the ``Graph`` class (:7-120) with the same
constructor arguments, ``init_graph``, ``warmup`` and ``capture_cuda_graph_qdrop`` (the captured
step: add weight noise, forward under bf16 autocast, loss, backward, remove the noise, clip the
gradient norm to 1, optimizer step), and the weight-noise helpers ``prepare_theta`` (:123-131),
``inject_noise`` (:133-145) and ``denoise`` (:163-170).

Platform specifics:
  * graphs are captured with ``keep_graph=True`` and, before instantiation, every memset node is
    rewritten into a kernel node by ``dopt_graph_replace_memsets``: replays of graphs holding
    memset nodes have given wrong results on this platform, and libraries record them on their
    own (torch's multi-block reductions clear their semaphores with hipMemsetAsync);
  * the compressed layers take every buffer from torch's allocator (the graph's private pool
    under capture) and never synchronise, so the whole step is one graph;
  * ``inject_noise`` computes the parameter and noise norms with one multi-tensor norm per list,
    not one reduction per parameter, and scales the noise in place in the ``_theta`` buffer,
    which then serves as the ``_noise`` the reference keeps in a second parameter-sized tensor.

Replay contract (as in the reference): the graph does not zero the gradients. Before each
replay, copy the batch into ``static_x`` / ``static_y`` and call
``opt.zero_grad(set_to_none=False)`` eagerly. The optimizer must be graph-safe
(``capturable=True`` for torch's Adam/AdamW). Quantizers with Philox stochastic rounding replay
the Philox offsets drawn at capture; nearest rounding (the default) has no state.

Behaviour kept from the reference: ``prepare_theta`` gives every trainable parameter a noise
buffer. Its BatchNorm2d test looks at the module of the outer loop, not at the parameter's
owner, so it excludes nothing whenever the model has any module that is not a BatchNorm2d.

``graph_module_in_place`` is the module-level counterpart: it turns one module's training
forward and backward into two replayed graphs (what the reference's Controller gets from
``torch.compile(mode='reduce-overhead')``, controller.py:316-331) and is what
``Controller.enable_graph_mode`` applies to the rewritten model.
"""
from __future__ import annotations

import ctypes

import torch
import torch.cuda as cuda
import torch.nn as nn

from ._lib import check, lib

NODE_TYPES = ("kernel", "memcpy", "memset", "host", "graph", "empty", "wait_event", "event_record",
              "ext_semaphore_signal", "ext_semaphore_wait", "mem_alloc", "mem_free", "memcpy_from_symbol",
              "memcpy_to_symbol", "batch_mem_op")


def _raw(g: torch.cuda.CUDAGraph) -> int:
    h = g.raw_cuda_graph()
    if not h:
        raise RuntimeError("the graph holds no captured hipGraph_t (construct it with keep_graph=True)")
    return h


def graph_node_counts(g: torch.cuda.CUDAGraph) -> dict:
    """Nodes of a captured graph (``keep_graph=True``) by type, child graphs included."""
    counts = (ctypes.c_int64 * len(NODE_TYPES))()
    check(lib().dopt_graph_node_counts(ctypes.c_void_p(_raw(g)), counts, len(NODE_TYPES)), "dopt_graph_node_counts")
    return {name: int(c) for name, c in zip(NODE_TYPES, counts) if c}


def replace_memset_nodes(g: torch.cuda.CUDAGraph) -> int:
    """Rewrites the memset nodes of a captured, not yet instantiated graph into fill-kernel nodes;
    returns how many there were."""
    n = ctypes.c_int64(0)
    check(lib().dopt_graph_replace_memsets(ctypes.c_void_p(_raw(g)), ctypes.byref(n)), "dopt_graph_replace_memsets")
    return int(n.value)


def finalize(g: torch.cuda.CUDAGraph) -> int:
    """Memset-free instantiation of a graph captured with ``keep_graph=True``."""
    n = replace_memset_nodes(g)
    g.instantiate()
    return n


class Graph:
    """cuda_graph_utils.py:7-120: captures ``num_of_graph`` copies of one training step."""

    def __init__(self, model: nn.Module, criterion: nn.Module, opt: torch.optim.Optimizer, data_loader,
                 stream: torch.cuda.Stream | None, mode: str, num_of_graph: int, device: str = "cuda"):
        self.model = model.to(device)
        self.criterion = criterion
        self.opt = opt
        self.data_loader = data_loader
        self.mode = mode
        self.num_of_graph = num_of_graph
        self.device = device
        self.compute_stream = cuda.Stream() if stream is None else stream
        self.cuda_graph_pool_handle = cuda.graph_pool_handle()
        self.graphs = [None] * num_of_graph
        self.memsets_replaced = [0] * num_of_graph
        x, y = next(iter(data_loader))
        self.static_x = torch.empty_like(x, device=device)
        self.static_y = torch.empty_like(y, device=device)
        prepare_theta(self.model)

    def init_graph(self):
        for i in range(self.num_of_graph):
            self.graphs[i] = cuda.CUDAGraph(keep_graph=True)

    def _step(self, clip: bool):
        inject_noise(self.model)
        logits = self.model(self.static_x)
        loss = self.criterion(logits, self.static_y)
        loss.backward()
        denoise(self.model)
        if clip:
            torch.nn.utils.clip_grad_norm_(self.model.parameters(), max_norm=1.0)
        self.opt.step()
        return logits, loss

    def warmup(self, empty: bool = False):
        """One eager step on the compute stream (:52-79), gradients zeroed afterwards."""
        self.compute_stream.wait_stream(cuda.current_stream())
        cuda.synchronize()
        x, y = next(iter(self.data_loader))
        with cuda.stream(self.compute_stream):
            with torch.amp.autocast(device_type="cuda", dtype=torch.bfloat16):
                self.static_x.copy_(x.to(self.device))
                self.static_y.copy_(y.to(self.device))
                self._step(clip=False)
                self.opt.zero_grad(set_to_none=False)
        cuda.current_stream().wait_stream(self.compute_stream)
        cuda.synchronize()
        if empty:
            cuda.empty_cache()

    def capture_cuda_graph_qdrop(self):
        """:82-120. Returns (graphs, compute_stream, static_x, static_y, logits, loss); the last two
        are the static outputs of the last graph captured, detached: they share the graph's output
        memory, so every replay refreshes them, but hold no reference to the captured autograd graph
        (which would keep its AccumulateGrad nodes, bound to the capture stream, alive)."""
        self.init_graph()
        self.warmup(empty=True)
        self.warmup()
        logits = loss = None
        for i in range(self.num_of_graph):
            g = self.graphs[i]
            cuda.current_stream().wait_stream(self.compute_stream)
            cuda.synchronize()
            self.opt.zero_grad(set_to_none=False)
            with cuda.stream(self.compute_stream):
                with cuda.graph(g):
                    with torch.amp.autocast(device_type="cuda", dtype=torch.bfloat16):
                        logits, loss = self._step(clip=True)
            logits, loss = logits.detach(), loss.detach()
            self.memsets_replaced[i] = finalize(g)
            cuda.synchronize()
        return self.graphs, self.compute_stream, self.static_x, self.static_y, logits, loss


def prepare_theta(model: nn.Module) -> None:
    """cuda_graph_utils.py:123-131: a noise buffer ``p._theta`` for every trainable parameter."""
    for p in model.parameters():
        if p.requires_grad and not hasattr(p, "_theta"):
            p._theta = torch.empty_like(p)


@torch.no_grad()
def inject_noise(model: nn.Module, alpha: float = 0.0375) -> None:
    """cuda_graph_utils.py:133-145: p += alpha * (|p| / |theta|) * theta, theta ~ U(-alpha, alpha),
    with |.| the L2 norm over the whole parameter; the noise stays in ``p._noise`` for denoise."""
    ps = [p for p in model.parameters() if hasattr(p, "_theta")]
    if not ps:
        return
    thetas = [p._theta for p in ps]
    for t in thetas:
        t.uniform_(-alpha, alpha)
    norm_p = torch._foreach_norm(ps)
    norm_t = torch._foreach_norm(thetas)
    for p, t, n_p, n_t in zip(ps, thetas, norm_p, norm_t):
        t.mul_(alpha * (n_p / n_t))
        p.add_(t)
        p._noise = t
        p._denoise = True


@torch.no_grad()
def denoise(model: nn.Module) -> None:
    """cuda_graph_utils.py:163-170: removes the noise inject_noise added."""
    for p in model.parameters():
        if hasattr(p, "_denoise"):
            p.sub_(p._noise)
            del p._denoise
            del p._noise


# -- module-level capture: the forward and the backward of one module as two replayed graphs ------


def _as_tuple(out):
    return out if isinstance(out, tuple) else (out,)


class _Capture:
    """The forward graph, the backward graph and their static buffers for one input signature."""

    def __init__(self, module: nn.Module, args, autocast, warmup_iters: int):
        forward = type(module).forward
        self.params = tuple(p for p in module.parameters() if p.requires_grad)
        self.static_in = tuple(a.detach().clone().requires_grad_(a.requires_grad) for a in args)
        diff_in = tuple(a for a in self.static_in if a.requires_grad) + self.params
        enabled, dtype = autocast

        def run():
            # the autocast weight cache is off: a cached cast made outside a graph would be replayed stale
            with torch.autocast("cuda", dtype=dtype, enabled=enabled, cache_enabled=False):
                out = forward(module, *self.static_in)
            self.tuple_out = isinstance(out, tuple)
            return _as_tuple(out)

        side = cuda.Stream()
        side.wait_stream(cuda.current_stream())
        with cuda.stream(side):
            for _ in range(warmup_iters):
                outs = [o for o in run() if o.requires_grad]
                torch.autograd.grad(outs, diff_in, grad_outputs=[torch.zeros_like(o) for o in outs],
                                    allow_unused=True)
                del outs
        cuda.current_stream().wait_stream(side)
        cuda.synchronize()

        self.fwd = cuda.CUDAGraph(keep_graph=True)
        self.bwd = cuda.CUDAGraph(keep_graph=True)
        with cuda.graph(self.fwd):
            outs = run()
        self.static_out = tuple(o.detach() for o in outs)
        self.out_requires_grad = tuple(o.requires_grad for o in outs)
        graded = [o for o in outs if o.requires_grad]
        self.static_grad_out = tuple(torch.empty_like(o) for o in graded)
        with cuda.graph(self.bwd, pool=self.fwd.pool()):
            grads = torch.autograd.grad(graded, diff_in, grad_outputs=self.static_grad_out, allow_unused=True)
        del outs, graded
        grads = iter(grads)
        self.static_grad_in = tuple(next(grads) if a.requires_grad else None for a in self.static_in) + \
            tuple(next(grads) for _ in self.params)
        self.memsets_replaced = finalize(self.fwd) + finalize(self.bwd)
        cuda.synchronize()


class _ReplayFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, cap: _Capture, *inputs):
        for s, x in zip(cap.static_in, inputs):
            if s.data_ptr() != x.data_ptr():
                s.copy_(x)
        cap.fwd.replay()
        ctx.cap = cap
        outs = tuple(o.detach() for o in cap.static_out)
        ctx.mark_non_differentiable(*(o for o, rg in zip(outs, cap.out_requires_grad) if not rg))
        return outs

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, *grads):
        cap = ctx.cap
        graded = (g for g, rg in zip(grads, cap.out_requires_grad) if rg)
        for static, g in zip(cap.static_grad_out, graded):
            if g is None:
                static.zero_()
            elif static.data_ptr() != g.data_ptr():
                static.copy_(g)
        cap.bwd.replay()
        return (None,) + tuple(None if g is None else g.detach() for g in cap.static_grad_in)


def graph_module_in_place(module: nn.Module, warmup_iters: int = 2) -> nn.Module:
    """Makes ``module``'s training forward and backward replay HIP graphs, in place.

    This is what the reference gets from ``module.compile(mode='reduce-overhead')``
    (Activation_Compression/controller.py:316-331): the module object, its parameters and its
    state dict stay the same; its ``forward`` becomes a replay. On the first training call with a
    given input signature (shapes, dtypes, autocast state) the module is run ``warmup_iters``
    times eagerly on a side stream, then its forward is captured into one graph and the gradient
    of its outputs with respect to its floating inputs and trainable parameters into a second,
    both in one memory pool, memset nodes rewritten into kernels (``finalize``). Later calls copy
    the inputs into the static input buffers and replay; the backward replays the second graph
    and hands the parameter gradients to autograd, which accumulates them into ``.grad`` as for
    any other function.

    Contract (the same as torch.cuda.make_graphed_callables'): a call's outputs live in static
    buffers that the next call overwrites, so run the backward of one call before the next
    forward; state a forward mutates outside its outputs (BatchNorm running statistics) is
    updated by each replay as in eager mode, and by the warm-up runs and the capture once each;
    hooks inside the module run at capture only. Calls without grad mode, in eval mode or with
    inputs not on the GPU run the eager forward.
    """
    if "forward" in vars(module):
        return module  # already graphed
    eager = type(module).forward
    captures = {}

    def forward(*args):
        tensors = all(isinstance(a, torch.Tensor) and a.is_cuda for a in args)
        if not (torch.is_grad_enabled() and module.training and tensors and args):
            return eager(module, *args)
        autocast = (torch.is_autocast_enabled("cuda"), torch.get_autocast_dtype("cuda"))
        key = (tuple((tuple(a.shape), a.dtype, a.requires_grad) for a in args), autocast)
        cap = captures.get(key)
        if cap is None:
            cap = captures[key] = _Capture(module, args, autocast, warmup_iters)
        outs = _ReplayFunction.apply(cap, *args, *cap.params)
        return outs if cap.tuple_out else outs[0]

    module.forward = forward
    module._dopt_graph_captures = captures
    return module


__all__ = ["Graph", "prepare_theta", "inject_noise", "denoise", "graph_node_counts", "replace_memset_nodes",
           "finalize", "graph_module_in_place", "NODE_TYPES"]
