"""Host mirror of the reference engine's linear path: the name-keyed weight
store, load-time fusion of projections, the bounded decoded-weight cache and
the `Engine::linear` dispatch (laoyin/a100-vision-infer src/engine.cpp:94-177,
196-242).

The decision table itself runs in the native library
(`fp8lin_engine_linear`, include/fp8lin.h); this class keeps the weights as
device tensors and hands them over as `fp8lin_weight` records, together with
the `name.bias` vector the native call adds (src/engine.cpp:240).  The
tensor-parallel reduce that the reference runs before the bias
(src/engine.cpp:239) needs a second GPU and is outside this path.
"""
import contextlib
import ctypes

import torch

from ._lib import (ERR_ARGUMENT, PATH_TENSOR_SMALL, Fp8linError, LinearOptions, Weight, check, lib)
from .ops import fp8_decode, fused_swiglu, qk_norm_rope


def check_options(options):
    """The linear-path option checks of the reference's Engine constructor
    (src/engine.cpp:78-81), with its messages."""
    if options.fp8_tensor_small and options.tilelang_fp8:
        raise Fp8linError(ERR_ARGUMENT, "Choose one FP8 Tensor Core backend")
    if options.fp8_tensor_split not in (1, 4):
        raise Fp8linError(ERR_ARGUMENT, "FP8 Tensor Core split must be 1 or 4")
    if (options.fp8_tensor_small or options.tilelang_fp8) and not options.optimized:
        raise Fp8linError(ERR_ARGUMENT, "FP8 Tensor Core requires optimized mode")


def profile_label(name):
    """The timing label of `Engine::linear` (src/engine.cpp:203)."""
    if name == "lm_head":
        return "linear.head"
    if name.startswith("model.visual."):
        return "linear.vision"
    if name.startswith("mtp."):
        return "linear.mtp"
    return "linear.text"


def cache_order(names, cache_vision_weights):
    """Fill order of the decoded-weight cache (src/engine.cpp:127-137): by
    name; with cache_vision_weights, MTP matrices first, then vision, then the
    rest, each run still by name."""
    names = sorted(names)
    if cache_vision_weights:
        def priority(n):
            return 0 if n.startswith("mtp.") else 1 if n.startswith("model.visual.") else 2
        names = sorted(names, key=priority)  # sorted() is stable
    return names


class StoredWeight:
    """`struct Weight { Tensor data, scale; }` (include/avi/engine.h:15)."""

    def __init__(self, data, scale=None):
        self.data = data
        self.scale = scale

    def compatible(self, other):
        # src/engine.cpp:154-158
        if self.data.dtype != other.data.dtype or (self.scale is None) != (other.scale is None):
            return False
        if self.scale is None:
            return True
        return self.scale.dim() == other.scale.dim() and (
            self.scale.dim() == 1 or self.scale.size(1) == other.scale.size(1))


class LinearEngine:
    """Options are the reference's `EngineOptions` linear flags
    (`LinearOptions`) plus `cache_vision_weights` (cache fill order),
    `profile_kernels` (per-label event timing, `profile_report`) and
    `reference_prefill` (`--reference-prefill`: fused weights keep views of
    their sources, and prefill steps run unoptimized; `step_mode`)."""

    def __init__(self, options=None, weight_cache_bytes=0, cache_vision_weights=False, profile_kernels=False,
                 reference_prefill=False):
        self.options = options or LinearOptions()
        check_options(self.options)
        self.weight_cache_bytes = int(weight_cache_bytes)
        self.cache_vision_weights = bool(cache_vision_weights)
        self.profile_kernels = bool(profile_kernels)
        self.reference_prefill = bool(reference_prefill)
        self.weights = {}
        self.biases = {}
        self.mixed_projections = {}
        self.decoded_weights = {}
        self.decoded_bytes = 0
        # include/avi/engine.h:78 (reported by Engine::cache_stats, src/engine.cpp:598)
        self.fp8_tensor_calls = 0
        self.tilelang_fp8_calls = 0
        self._profile_events = []
        self._workspaces = {}

    # -- loading -------------------------------------------------------------
    def add(self, name, data, scale=None):
        """Register `name` (e.g. "...mlp.gate_proj.weight") with device
        tensors: uint8 codes [N,K] + float32 scales, or BF16 [N,K]; or a
        BF16 bias vector [N] under "....bias"."""
        if name.endswith(".bias") and data.dim() == 1:
            if data.dtype != torch.bfloat16 or scale is not None:
                raise Fp8linError(ERR_ARGUMENT, f"Bias {name} must be an unquantized BF16 vector")
            self.biases[name] = data.contiguous()
            return
        if data.dim() != 2 or not data.is_contiguous():
            raise Fp8linError(ERR_ARGUMENT, f"Invalid matrix {name}")
        self.weights[name] = StoredWeight(data, scale)

    def fuse_weights(self, dest, sources):
        """Row-concatenate compatible projections (src/engine.cpp:147-177):
        `dest.weight = cat(sources)`; incompatible runs (e.g. FP8 qkv+z next
        to BF16 b+a) become groups whose outputs are concatenated."""
        ws = [self.weights[s + ".weight"] for s in sources]
        scaled = [w for w in ws if w.scale is not None]
        mixed = scaled and (len(scaled) != len(ws) or any(
            w.scale.dim() != scaled[0].scale.dim() or
            (w.scale.dim() == 2 and w.scale.size(1) != scaled[0].scale.size(1)) for w in scaled))
        if mixed:
            groups = []
            for s in sources:
                if not groups or not self.weights[groups[-1][-1] + ".weight"].compatible(
                        self.weights[s + ".weight"]):
                    groups.append([])
                groups[-1].append(s)
            children = []
            for i, g in enumerate(groups):
                if len(g) == 1:
                    children.append(g[0])
                    continue
                child = f"{dest}.group{i}"
                self.fuse_weights(child, g)
                children.append(child)
            self.mixed_projections[dest] = children
            return
        data = torch.cat([w.data for w in ws], 0)
        scale = torch.cat([w.scale for w in ws], 0) if scaled else None
        self.weights[dest + ".weight"] = StoredWeight(data, scale)
        offset = 0
        for s, w in zip(sources, ws):
            rows = w.data.size(0)
            if self.reference_prefill:
                # src/engine.cpp:172-173: the source name stays, as a view of
                # its rows of the fused weight (no second allocation), for the
                # unoptimized prefill steps
                self.weights[s + ".weight"] = StoredWeight(
                    data.narrow(0, offset, rows), scale.narrow(0, offset, rows) if scale is not None else None)
            else:
                del self.weights[s + ".weight"]
            offset += rows

    def cache_candidates(self):
        """The matrices the reference may cache (src/engine.cpp:130-132):
        quantized layer and MTP matrices, and 2-D vision matrices when
        cache_vision_weights is set."""
        return [n for n, w in self.weights.items() if w.scale is not None and (
            n.startswith("model.language_model.layers.") or n.startswith("mtp.") or
            (self.cache_vision_weights and n.startswith("model.visual.") and w.data.dim() == 2))]

    def build_cache(self, names=None):
        """Bounded decoded-BF16 cache (src/engine.cpp:127-143): `names` (every
        quantized matrix when None) in cache_order, each decoded while it fits
        in what is left of weight_cache_bytes."""
        if names is None:
            names = [n for n, w in self.weights.items() if w.scale is not None]
        for name in cache_order(names, self.cache_vision_weights):
            w = self.weights[name]
            nbytes = w.data.numel() * 2
            if nbytes <= self.weight_cache_bytes - self.decoded_bytes:
                self.decoded_weights[name] = fp8_decode(w.data, w.scale)
                self.decoded_bytes += nbytes

    @staticmethod
    def qkv_gate_views(projected, heads, kv_heads, head_dim):
        """The fused QKV-gate output [T, H*2D + 2*HK*D] split as the reference
        slices it (src/engine.cpp:279-282): q [T,H,D] and gate [T,H*D] from the
        per-head [q | gate] rows, k and v [T,HK,D].  q, k and v are views; gate
        is a reshape of a strided view, which copies, as in the reference."""
        T, D, H, HK = projected.size(0), head_dim, heads, kv_heads
        if projected.size(-1) != H * 2 * D + 2 * HK * D:
            raise Fp8linError(ERR_ARGUMENT, "QKV-gate output width does not match the head layout")
        qg = projected.narrow(-1, 0, H * 2 * D).reshape(T, H, 2 * D)
        q = qg.narrow(-1, 0, D)
        gate = qg.narrow(-1, D, D).reshape(T, H * D)
        k = projected.narrow(-1, H * 2 * D, HK * D).reshape(T, HK, D)
        v = projected.narrow(-1, H * 2 * D + HK * D, HK * D).reshape(T, HK, D)
        return q, gate, k, v

    def full_attention_inputs(self, x, prefix, positions, q_norm, k_norm, heads, kv_heads, head_dim, rope, eps):
        """The projection and Q/K epilogue of `Engine::full_attention`, optimized
        branch (src/engine.cpp:276-287): projected = linear(x, prefix.qkv_gate);
        q and k are RMS-normalised per head (centered, q_norm / k_norm) and
        rotated by the interleaved mRoPE of `rope` (the model config's
        rope_parameters: partial_rotary_factor, mrope_section, rope_theta), in
        one launch; gate and v are as in qkv_gate_views.  Returns
        (q [T,H,D], gate [T,H*D], k [T,HK,D], v [T,HK,D])."""
        projected = self.linear(x, prefix + ".qkv_gate")
        _, gate, _, v = self.qkv_gate_views(projected, heads, kv_heads, head_dim)
        rotary = int(head_dim * rope.get("partial_rotary_factor", 0.25))
        sections = rope["mrope_section"]
        q, k = qk_norm_rope(projected, q_norm, k_norm, positions, heads, kv_heads, head_dim, rotary,
                            rope["rope_theta"], sections[1], sections[2], eps)
        return q, gate, k, v

    # -- steps -----------------------------------------------------------------
    @contextlib.contextmanager
    def step_mode(self, decode=False, verifying=False):
        """The option override of `Engine::step` (src/engine.cpp:403-405):
        with reference_prefill, a prefill step (neither decode nor MTP
        verification) runs with `optimized` off and restores it on exit."""
        saved = self.options.optimized
        if self.reference_prefill and not decode and not verifying:
            self.options.optimized = 0
        try:
            yield self
        finally:
            self.options.optimized = saved

    def mlp(self, n, prefix):
        """The MLP of `Engine::step` (src/engine.cpp:415-416) on one rank:
        optimized, `fused_swiglu(linear(n, gate_up))`; otherwise the unfused
        `silu(linear(n, gate_proj)) * linear(n, up_proj)` on the source
        weights, with the same two BF16 rounding points (the SwiGLU of the two
        outputs side by side).  Then `linear(gated, down_proj)`; the
        cross-rank reduce is the caller's."""
        if self.options.optimized:
            gated = fused_swiglu(self.linear(n, prefix + ".gate_up"))
        else:
            gate = self.linear(n, prefix + ".gate_proj")
            up = self.linear(n, prefix + ".up_proj")
            rows = gate.numel() // gate.size(-1)
            pair = torch.cat([gate.reshape(rows, -1), up.reshape(rows, -1)], -1)
            gated = fused_swiglu(pair).reshape(*gate.shape)
        return self.linear(gated, prefix + ".down_proj")

    # -- dispatch --------------------------------------------------------------
    def _record(self, name):
        w = self.weights.get(name + ".weight")
        if w is None:
            raise Fp8linError(ERR_ARGUMENT, f"Missing linear {name}")
        cached = self.decoded_weights.get(name + ".weight")
        rec = Weight()
        rec.data = w.data.data_ptr()
        rec.scales = w.scale.data_ptr() if w.scale is not None else None
        rec.scale_cols = (1 if w.scale.dim() == 1 else w.scale.size(1)) if w.scale is not None else 1
        rec.cached_bf16 = cached.data_ptr() if cached is not None else None
        rec.N, rec.K = w.data.size(0), w.data.size(1)
        bias = self.biases.get(name + ".bias")
        if bias is not None and bias.numel() != rec.N:
            raise Fp8linError(ERR_ARGUMENT, f"Bias of {name} does not match its {rec.N} output rows")
        rec.bias = bias.data_ptr() if bias is not None else None
        return rec

    def _ws(self, nbytes, device):
        """Workspace for one call on torch's current stream.  Outside graph
        capture each stream keeps its own buffer (concurrent calls on other
        streams never share one), grown by replacement.  During capture the
        call gets a fresh buffer from the capture's private pool, which the
        graph keeps for its replays, so a later larger eager call can never
        free memory that a graph still writes."""
        if nbytes == 0:
            return None
        if torch.cuda.is_current_stream_capturing():
            return torch.empty(nbytes, dtype=torch.uint8, device=device)
        key = torch.cuda.current_stream(device).cuda_stream
        ws = self._workspaces.get(key)
        if ws is None or ws.numel() < nbytes:
            ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
            self._workspaces[key] = ws
        return ws

    def _count(self, path):
        # src/engine.cpp:211-212
        if path == PATH_TENSOR_SMALL:
            if self.options.tilelang_fp8:
                self.tilelang_fp8_calls += 1
            else:
                self.fp8_tensor_calls += 1

    def _profile_begin(self, name, device):
        if not self.profile_kernels:
            return None
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(torch.cuda.current_stream(device))
        self._profile_events.append((profile_label(name), start, end))
        return end

    def _profile_end(self, end, device):
        if end is not None:
            end.record(torch.cuda.current_stream(device))

    def profile_report(self):
        """{label: {"calls", "cuda_ms"}} over the calls since the last report
        (Engine::profile_report, src/engine.cpp:34-43); {} unless
        profile_kernels."""
        report = {}
        if not self.profile_kernels:
            return report
        torch.cuda.synchronize()
        for label, start, end in self._profile_events:
            row = report.setdefault(label, {"calls": 0, "cuda_ms": 0.0})
            row["calls"] += 1
            row["cuda_ms"] += start.elapsed_time(end)
        self._profile_events.clear()
        return report

    def cache_stats(self):
        """The linear-path entries of Engine::cache_stats (src/engine.cpp:598)."""
        return {"fp8_tensor_calls": self.fp8_tensor_calls, "tilelang_fp8_calls": self.tilelang_fp8_calls}

    def local_candidates(self, x, name="lm_head", offset=0, return_path=False):
        """`Engine::local_candidates` with gpu_candidates (src/speculative.cpp:25-27):
        the projection through this engine's dispatch, then per row the
        {max value, argmax + offset} pair as doubles [rows, 2]."""
        rows = x.numel() // x.size(-1)
        x2 = x.reshape(rows, x.size(-1)).contiguous()
        rec = self._record(name)
        opt = self.options
        out = torch.empty((rows, 2), dtype=torch.float64, device=x.device)
        need = lib().fp8lin_engine_linear_candidates_workspace_bytes(ctypes.byref(opt), ctypes.byref(rec), rows)
        ws = self._ws(need, x.device)
        path = ctypes.c_int(0)
        stream = ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)
        end = self._profile_begin(name, x.device)
        check(lib().fp8lin_engine_linear_candidates(
            ctypes.byref(opt), ctypes.byref(rec), ctypes.c_void_p(x2.data_ptr()), rows, int(offset),
            ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(ws.data_ptr()) if ws is not None else None, need,
            ctypes.byref(path), stream))
        self._profile_end(end, x.device)
        self._count(path.value)
        return (out, path.value) if return_path else out

    def linear(self, x, name, return_path=False):
        """`Engine::linear(x, name)` on one rank (src/engine.cpp:196-242): the
        branch, then the `name.bias` add; the cross-rank reduce is not run."""
        rows = x.numel() // x.size(-1)
        x2 = x.reshape(rows, x.size(-1)).contiguous()
        stream = ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)
        opt = self.options
        if name in self.mixed_projections:
            recs = [self._record(c) for c in self.mixed_projections[name]]
            total = sum(r.N for r in recs)
            y = torch.empty((rows, total), dtype=torch.bfloat16, device=x.device)
            need = max(lib().fp8lin_engine_linear_workspace_bytes(ctypes.byref(opt), ctypes.byref(r),
                                                                  rows) for r in recs)
            ws = self._ws(need, x.device)
            arr = (Weight * len(recs))(*recs)
            check(lib().fp8lin_engine_linear_groups(
                ctypes.byref(opt), arr, len(recs), ctypes.c_void_p(x2.data_ptr()), rows,
                ctypes.c_void_p(y.data_ptr()), total,
                ctypes.c_void_p(ws.data_ptr()) if ws is not None else None, need, stream))
            for r in recs:
                self._count(lib().fp8lin_engine_linear_path(ctypes.byref(opt), ctypes.byref(r), rows))
            out = y.reshape(*x.shape[:-1], total)
            return (out, None) if return_path else out
        rec = self._record(name)
        y = torch.empty((rows, rec.N), dtype=torch.bfloat16, device=x.device)
        need = lib().fp8lin_engine_linear_workspace_bytes(ctypes.byref(opt), ctypes.byref(rec), rows)
        ws = self._ws(need, x.device)
        path = ctypes.c_int(0)
        end = self._profile_begin(name, x.device)
        check(lib().fp8lin_engine_linear(
            ctypes.byref(opt), ctypes.byref(rec), ctypes.c_void_p(x2.data_ptr()), rows,
            ctypes.c_void_p(y.data_ptr()), rec.N,
            ctypes.c_void_p(ws.data_ptr()) if ws is not None else None, need,
            ctypes.byref(path), stream))
        self._profile_end(end, x.device)
        self._count(path.value)
        out = y.reshape(*x.shape[:-1], rec.N)
        return (out, path.value) if return_path else out
