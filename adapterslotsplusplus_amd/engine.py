"""WarpPipeEngine -- the drop-in Python surface of the grouped multi-LoRA apply.

Mirrors lora_warp_pipe/engine.py:7-69 of the reference (same method names,
argument order, return conventions and errors) on top of the MI355X C ABI
(include/warppipe_mi355x.h, libwarppipe_mi355x.so).  PyTorch provides device
memory and the current stream; all compute is in the library's HIP kernels.

Conventions kept from the reference:
  * errors raise RuntimeError (TORCH_CHECK / std::runtime_error there);
  * "cannot handle" returns False (build_seg_bounds above capacity,
    add_lora_packed for a rank without kernels) or -1 (prefetch_adapter);
  * compute is enqueued on torch's current stream, prefetch on a private stream;
  * shrink() returns a new zero-initialised H [T, rank]; expand() updates Y in place.

Additions (each a superset of the reference behaviour):
  * fp16 and bf16, ranks 8/16/32/64 on every path (the reference: fp16 only;
    add_lora_packed and build_seg_bounds rank 32 only);
  * shrink/expand also run on a build_seg_bounds table, through the adapter
    store (the reference reads stale pointers there);
  * rank=0 in shrink/expand selects mixed ranks (each adapter's own rank);
  * add_lora_packed takes y_offset / y_slice_size; add_lora_slices expands
    into several output slices in one launch, from one shared A or one A per
    slice (add_lora_packed_nslice, vLLM's packed q/k/v and gate/up layers);
  * register_adapter with CPU tensors puts the adapter in the pinned host
    store; prefetch_adapter then stages it in HBM.
"""
from __future__ import annotations

import ctypes
from typing import List, Optional, Sequence, Tuple

import torch

from . import _lib
from .config import WarpPipeConfig

_DTYPES = {torch.float16: _lib.WP_DTYPE_F16, torch.bfloat16: _lib.WP_DTYPE_BF16}


def _dtype_code(t: torch.Tensor, what: str) -> int:
    code = _DTYPES.get(t.dtype)
    if code is None:
        raise RuntimeError(f"{what} must be fp16 or bf16, got {t.dtype}")
    return code


def _ptr(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def _current_raw_stream(device_index: int) -> int:
    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is not None:
        return int(raw(device_index))
    return int(torch.cuda.current_stream(device_index).cuda_stream)


class _Ext:
    """Stand-in for the reference's `engine._ext` extension object: exposes the
    free functions tests call on it (test_rank_variants.py:97-103)."""

    def __init__(self, lib):
        self._lib = lib

    def rank_supported(self, rank: int) -> bool:
        return bool(self._lib.wp_rank_supported(int(rank)))


class WarpPipeEngine:
    def __init__(self, config: Optional[WarpPipeConfig] = None):
        self.config = config or WarpPipeConfig()
        self._lib = _lib.load()
        self._ext = _Ext(self._lib)
        self._handle = ctypes.c_void_p(None)
        dev = self.config.device
        if dev is None:
            if not torch.cuda.is_available():
                raise RuntimeError("WarpPipeEngine: no GPU available (the apply runs only on the GPU)")
            dev = torch.cuda.current_device()
        self.device = torch.device("cuda", int(dev))
        self._dev_index = int(dev)
        self._ranks = {}  # rank -> the library's rank_supported answer
        cfg = _lib.WpConfig(int(dev), int(self.config.num_staging_slots), int(self.config.max_tokens), 64,
                            int(self.config.max_adapter_ids))
        _lib.check(self._lib.wp_create(ctypes.byref(cfg), ctypes.byref(self._handle)), "WarpPipeEngine")
        self._held = {}
        self._layers = {}  # adapter id -> layers registered under it (multi-layer store)

    # ----------------------------------------------------- adapter layers --
    def _store_id(self, adapter_id, layer) -> int:
        """The store's id for (adapter_id, layer): adapter_id itself for layer
        None / 0 without a layer stride, else layer * stride + adapter_id."""
        aid = int(adapter_id)
        stride = int(self.config.layer_stride or 0)
        if stride <= 0:
            if layer not in (None, 0):
                raise RuntimeError("adapter layers need WarpPipeConfig.layer_stride > 0")
            return aid
        lay = int(layer or 0)
        if not 0 <= aid < stride or lay < 0:
            raise RuntimeError(f"with layer_stride {stride}, adapter ids must be in [0, {stride}) and layers >= 0")
        sid = lay * stride + aid
        if sid >= 2 ** 31:
            raise RuntimeError("layer * layer_stride + adapter_id exceeds the int32 id range")
        return sid

    def _select_layer(self, layer) -> None:
        stride = int(self.config.layer_stride or 0)
        if layer not in (None, 0) and stride <= 0:
            raise RuntimeError("adapter layers need WarpPipeConfig.layer_stride > 0")
        if layer is not None and int(layer) < 0:
            raise RuntimeError("layer must be >= 0")
        _lib.check(self._lib.wp_set_entry_offset(self._handle, int(layer or 0) * stride, stride), "layer")

    # ------------------------------------------------------------ lifetime --
    def close(self) -> None:
        h = getattr(self, "_handle", None)
        if h is not None and h.value:
            self._lib.wp_destroy(h)
            self._handle = ctypes.c_void_p(None)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _stream(self) -> ctypes.c_void_p:
        # The raw handle of torch's current stream on the engine's device,
        # without building a torch.cuda.Stream object per call.
        return ctypes.c_void_p(_current_raw_stream(self._dev_index))

    def _on_device(self, t: torch.Tensor, what: str) -> None:
        # get_device() is an int (-1 on the CPU): cheaper per call than
        # building and comparing torch.device objects.
        dev = t.get_device()
        if dev != self._dev_index:
            if dev < 0:
                raise RuntimeError(f"{what} must be a CUDA tensor")
            raise RuntimeError(f"{what} is on {t.device}, the engine on {self.device}")

    # ------------------------------------------------------- adapter store --
    def register_adapter(self, adapter_id, A, B, alpha_scale, rank=None, layer=None, copy=True):
        """A [rank, d], B [o, rank], contiguous fp16/bf16 (reference engine.py:12-14,
        bindings:110-119).  CUDA tensors: the adapter is device-resident.  CPU
        tensors: it goes to the pinned host store and is usable once prefetched.
        layer (multi-layer store, config.layer_stride > 0): the layer these
        weights belong to.  copy=False (CUDA tensors only): the store keeps
        the tensors themselves, as the reference's pointer registry does
        (adapter_store.h:21-27) -- no copy, in-place updates to them are seen
        by later calls; the engine holds a reference to them until eviction."""
        sid = self._store_id(adapter_id, layer)
        rank = int(rank or self.config.rank)
        if A.is_cuda != B.is_cuda:
            raise RuntimeError("A/B must both be CUDA tensors or both CPU tensors")
        if A.is_cuda:
            self._on_device(A, "A")
            self._on_device(B, "B")
        if A.dtype != B.dtype:
            raise RuntimeError("A/B must have the same dtype")
        dt = _dtype_code(A, "A/B")
        if not (A.is_contiguous() and B.is_contiguous()):
            raise RuntimeError("A/B must be contiguous")
        d_model = int(A.size(-1))
        out_features = int(B.size(-2)) if B.dim() >= 2 else 0
        if A.numel() != rank * d_model or B.numel() != out_features * rank or int(B.size(-1)) != rank:
            raise RuntimeError(
                f"A must be [rank={rank}, d] and B [o, rank={rank}]; got {tuple(A.shape)} and {tuple(B.shape)}")
        host = 0 if A.is_cuda else 1
        if not copy:
            if host:
                raise RuntimeError("register_adapter(copy=False) needs CUDA tensors")
            _lib.check(self._lib.wp_register_adapter_ref(self._handle, sid, _ptr(A), _ptr(B), rank, d_model,
                                                         out_features, float(alpha_scale), dt, self._stream()),
                       "register_adapter")
        else:
            _lib.check(self._lib.wp_register_adapter(self._handle, sid, _ptr(A), _ptr(B), rank, d_model,
                                                     out_features, float(alpha_scale), dt, host, self._stream()),
                       "register_adapter")
        # Keeps the source alive until the stream-ordered copy has run (the
        # reference holds the tensors until eviction as well, bindings:118).
        self._held[sid] = (A, B) if host == 0 else None
        self._layers.setdefault(int(adapter_id), set()).add(int(layer or 0))

    def evict_adapter(self, adapter_id, layer=None):
        """Silent for an unknown id.  With a layer stride and layer=None, every
        layer registered under the id is evicted."""
        if int(self.config.layer_stride or 0) > 0 and layer is None:
            layers = sorted(self._layers.pop(int(adapter_id), {0}))
        else:
            layers = [layer]
            self._layers.get(int(adapter_id), set()).discard(int(layer or 0))
        for lay in layers:
            sid = self._store_id(adapter_id, lay)
            _lib.check(self._lib.wp_evict_adapter(self._handle, sid, self._stream()), "evict_adapter")
            self._held.pop(sid, None)

    # ------------------------------------------------------ segment tables --
    def build_segments(self, sorted_adapter_ids, seg_offsets):
        ids = [int(v) for v in sorted_adapter_ids]
        offs = [int(v) for v in seg_offsets]
        ids_c = (ctypes.c_int32 * max(len(ids), 1))(*ids)
        offs_c = (ctypes.c_int32 * max(len(offs), 1))(*offs)
        _lib.check(self._lib.wp_build_segments(self._handle, ids_c, len(ids), offs_c, len(offs), self._stream()),
                   "build_segments")

    def build_seg_bounds(self, token_lora_indices) -> bool:
        """Builds the step's segment table on the GPU; False iff the token count
        exceeds config.max_tokens (reference: engine.py:28-32, bindings:162-170)."""
        idx = token_lora_indices
        if not isinstance(idx, torch.Tensor) or not idx.is_cuda:
            raise RuntimeError("build_seg_bounds: token_lora_indices must be a CUDA tensor")
        self._on_device(idx, "token_lora_indices")
        if idx.dtype not in (torch.int64, torch.int32):
            idx = idx.to(torch.int64)
        idx = idx.reshape(-1)
        if not idx.is_contiguous():
            idx = idx.contiguous()
        T = int(idx.numel())
        rc = _lib.check(self._lib.wp_build_seg_bounds(self._handle, _ptr(idx), 1 if idx.dtype == torch.int64 else 0,
                                                      T, self._stream()), "build_seg_bounds")
        return rc == _lib.WP_OK

    def read_segments(self) -> List[Tuple[int, int, int]]:
        """The current segment table as (adapter_id, token_start, token_count)
        tuples (synchronises the current stream; for tests and debugging)."""
        cap = max(int(self.config.max_tokens), 256)
        buf = (ctypes.c_int32 * (3 * cap))()
        n = ctypes.c_int64(0)
        _lib.check(self._lib.wp_read_segments(self._handle, buf, cap, ctypes.byref(n), self._stream()),
                   "read_segments")
        m = min(n.value, cap)
        return [(buf[3 * i], buf[3 * i + 1], buf[3 * i + 2]) for i in range(m)]

    def read_plan(self):
        """(perm, blocks) of the current plan: the token order grouped by
        adapter and the (adapter_id, first, count, entry) work blocks."""
        cap = int(self.config.max_tokens)
        bcap = cap + 256
        perm = (ctypes.c_int32 * cap)()
        blocks = (ctypes.c_int32 * (4 * bcap))()
        nv = ctypes.c_int64(0)
        nb = ctypes.c_int64(0)
        _lib.check(self._lib.wp_read_plan(self._handle, perm, cap, blocks, bcap, ctypes.byref(nv), ctypes.byref(nb),
                                          self._stream()), "read_plan")
        return (list(perm[: min(nv.value, cap)]),
                [tuple(blocks[4 * i: 4 * i + 4]) for i in range(min(nb.value, bcap))])

    def device_errors(self) -> int:
        """Reads and clears the device error word (adapters the kernels had to
        skip: 1 id out of range, 2 unregistered, 4 shape mismatch; 8 a fused
        call's wait gave up; 16 shrink()/expand() found more blocks than the
        registered adapters allow, i.e. the routing names unregistered ids)."""
        v = ctypes.c_uint32(0)
        _lib.check(self._lib.wp_read_device_errors(self._handle, ctypes.byref(v), self._stream()), "device_errors")
        return int(v.value)

    def poll_device_errors(self) -> int:
        """The device error word without a host wait (not in the reference):
        returns the bits an earlier poll moved out of the word if that move
        has completed (else 0: they come with a later poll or with
        device_errors()), then enqueues the next move on torch's current
        stream.  For serving loops, once per step outside graph capture; a
        no-op returning 0 while the stream is capturing."""
        v = ctypes.c_uint32(0)
        _lib.check(self._lib.wp_poll_device_errors(self._handle, ctypes.byref(v), self._stream()),
                   "poll_device_errors")
        return int(v.value)

    def set_max_adapters(self, n: Optional[int]) -> None:
        """Declares the most adapters that will be registered at once (not in
        the reference; None or 0 withdraws the declaration).  Adapter-store
        calls (shrink / expand / shrink_expand / shrink_expand_slices on a
        build_seg_bounds table) captured into a graph then size their grids by
        n instead of by every id of the table, and registering an (n+1)-th
        adapter raises."""
        _lib.check(self._lib.wp_set_max_adapters(self._handle, int(n or 0)), "set_max_adapters")

    # --------------------------------------------------------------- apply --
    def shrink(self, X, d_model, rank, total_tokens, out=None, layer=None):
        """H = rn(alpha * X . A^T) per segment; returns a new zero-initialised
        [total_tokens, rank] tensor (reference bindings:132-139).  rank=0 or
        None: mixed ranks, H is [T, 64] with each row's first r_a columns set.
        `out` (not in the reference): a caller-owned [T, width] H to write
        instead; rows outside every segment keep their contents.  `layer`:
        the adapters' layer in a multi-layer store (build_seg_bounds tables)."""
        rank = int(rank or 0)
        self._on_device(X, "X")
        dt = _dtype_code(X, "X")
        if not X.is_contiguous():
            raise RuntimeError("X must be contiguous")
        T = int(total_tokens)
        if X.numel() < T * int(d_model):
            raise RuntimeError(f"X has {X.numel()} elements, fewer than total_tokens x d_model")
        width = rank if rank else 64
        if out is None:
            H = torch.zeros(T, width, dtype=X.dtype, device=X.device)
        else:
            H = out
            self._on_device(H, "out")
            if H.dtype != X.dtype or not H.is_contiguous() or tuple(H.shape) != (T, width):
                raise RuntimeError(f"out must be a contiguous [{T}, {width}] tensor of X's dtype")
        self._select_layer(layer)
        _lib.check(self._lib.wp_shrink(self._handle, _ptr(X), _ptr(H), int(d_model), rank, T, width, dt,
                                       self._stream()), "shrink")
        return H

    def expand(self, H, Y, out_features, rank, y_offset: int = 0, layer=None):
        """Y[:, y_offset:y_offset+o] += H . B^T per segment, in place
        (reference bindings:141-148); `layer` as for shrink()."""
        rank = int(rank or 0)
        self._on_device(H, "H")
        self._on_device(Y, "Y")
        if H.dtype != Y.dtype:
            raise RuntimeError("H/Y must have the same dtype")
        dt = _dtype_code(Y, "Y")
        if not (H.is_contiguous() and Y.is_contiguous()):
            raise RuntimeError("H/Y must be contiguous")
        if H.dim() != 2 or Y.dim() != 2:
            raise RuntimeError("expand: H and Y must be 2-D ([T, rank] and [T, width])")
        T = int(Y.size(0))
        # The library checks the table against Y's rows; H is read at the same
        # token rows, so it needs at least as many.
        if int(H.size(0)) < T:
            raise RuntimeError(f"expand: H has {int(H.size(0))} rows, Y has {T}")
        self._select_layer(layer)
        _lib.check(self._lib.wp_expand(self._handle, _ptr(H), _ptr(Y), int(out_features), rank, T, int(H.size(-1)),
                                       int(Y.size(-1)), int(y_offset), dt, self._stream()), "expand")

    def shrink_expand(self, X, Y, out_features, rank, y_offset: int = 0, layer=None):
        """shrink() then expand() as one call (not in the reference):
        Y[:, y_offset:y_offset+o] += rn(alpha * X . A^T) . B^T per segment, in
        place.  Decode-sized plans run in one launch with no H round trip
        (rank=0: mixed ranks); larger plans run the two halves through the
        engine's own H."""
        rank = int(rank or 0)
        self._on_device(X, "X")
        self._on_device(Y, "Y")
        if X.dim() != 2 or Y.dim() != 2:
            raise RuntimeError("shrink_expand: X and Y must be 2-D ([T, d] and [T, width])")
        if X.dtype != Y.dtype:
            raise RuntimeError("X/Y must have the same dtype")
        dt = _dtype_code(Y, "Y")
        if not (X.is_contiguous() and Y.is_contiguous()):
            raise RuntimeError("X/Y must be contiguous")
        if X.size(0) != Y.size(0):
            raise RuntimeError("X and Y have different token counts")
        self._select_layer(layer)
        _lib.check(self._lib.wp_shrink_expand(self._handle, _ptr(X), _ptr(Y), int(X.size(-1)), int(out_features), rank,
                                              int(Y.size(0)), int(Y.size(-1)), int(y_offset), dt, self._stream()),
                   "shrink_expand")

    def shrink_expand_slices(self, X, Y, layers, out_features, y_offsets, rank=0):
        """shrink_expand over several layers of the multi-layer store in one
        launch (not in the reference): slice i applies layer layers[i]'s
        adapter of each token's id into columns [y_offsets[i], + out_features[i])
        of Y, in place; X is read once (packed gate/up, for instance).  rank=0:
        each adapter at its registered rank."""
        rank = int(rank or 0)
        self._on_device(X, "X")
        self._on_device(Y, "Y")
        if X.dim() != 2 or Y.dim() != 2:
            raise RuntimeError("shrink_expand_slices: X and Y must be 2-D ([T, d] and [T, width])")
        if X.dtype != Y.dtype:
            raise RuntimeError("X/Y must have the same dtype")
        dt = _dtype_code(Y, "Y")
        if not (X.is_contiguous() and Y.is_contiguous()):
            raise RuntimeError("X/Y must be contiguous")
        if X.size(0) != Y.size(0):
            raise RuntimeError("X and Y have different token counts")
        n = len(layers)
        if len(out_features) != n or len(y_offsets) != n:
            raise RuntimeError("shrink_expand_slices: one width and one offset per layer")
        stride = int(self.config.layer_stride or 0)
        offs = (ctypes.c_int32 * max(n, 1))(*[self._store_id(0, int(l)) for l in layers])
        o_arr = (ctypes.c_int32 * max(n, 1))(*[int(o) for o in out_features])
        y_arr = (ctypes.c_int32 * max(n, 1))(*[int(v) for v in y_offsets])
        _lib.check(self._lib.wp_shrink_expand_slices(self._handle, _ptr(X), _ptr(Y), int(X.size(-1)), n, offs, stride,
                                                     o_arr, y_arr, rank, int(Y.size(0)), int(Y.size(-1)), dt,
                                                     self._stream()), "shrink_expand_slices")

    def linear_lora(self, x, weight, bias, wa_t_all, wb_t_all, scale, out=None):
        """The base linear and its per-token LoRA delta in one launch (not in the
        reference, whose draft wrapper runs F.linear and then bgmv_shrink /
        bgmv_expand into its output, serve_multitenant.py:56-87):
        y = rn(rn(x . W^T + bias) + rn(scale . x . A[idx]^T) . B[idx]^T) over
        the last build_seg_bounds table.  x [T, in]; weight [out, in]; bias
        [out] or None; wa_t_all [L, 1, r, in], wb_t_all [L, 1, out, r].
        Returns y ([T, out], new unless `out` is given), or None when the
        shapes have no kernel (the caller then runs F.linear and
        add_lora_packed)."""
        self._on_device(x, "x")
        self._on_device(weight, "weight")
        for t, nm in ((wa_t_all, "wa_t_all"), (wb_t_all, "wb_t_all")):
            self._on_device(t, nm)
        dt = _dtype_code(x, "x")
        if weight.dtype != x.dtype or wa_t_all.dtype != x.dtype or wb_t_all.dtype != x.dtype or (
                bias is not None and bias.dtype != x.dtype):
            raise RuntimeError("linear_lora: x, weight, bias and the LoRA weights must share one dtype")
        x2 = x.reshape(-1, x.size(-1))
        if not x2.is_contiguous() or not wa_t_all.is_contiguous() or not wb_t_all.is_contiguous():
            raise RuntimeError("linear_lora: x and the LoRA weights must be contiguous")
        if weight.dim() != 2 or weight.stride(1) != 1:
            raise RuntimeError("linear_lora: weight must be [out, in] with unit column stride")
        T, d_in = int(x2.size(0)), int(x2.size(1))
        d_out = int(weight.size(0))
        rank = int(wb_t_all.size(-1))
        L = int(wa_t_all.size(0))
        if int(weight.size(1)) != d_in or int(wa_t_all.size(-1)) != d_in or int(wa_t_all.size(-2)) != rank:
            raise RuntimeError("linear_lora: weight / wa_t_all do not match x's width")
        if int(wb_t_all.size(0)) != L or int(wb_t_all.size(-2)) != d_out:
            raise RuntimeError("linear_lora: wb_t_all must be [L, 1, out, r]")
        if bias is not None:
            self._on_device(bias, "bias")
            if bias.numel() != d_out or not bias.is_contiguous():
                raise RuntimeError("linear_lora: bias must be a contiguous [out] tensor")
        y = out if out is not None else torch.empty(T, d_out, dtype=x.dtype, device=x.device)
        self._on_device(y, "out")
        if tuple(y.shape) != (T, d_out) or not y.is_contiguous() or y.dtype != x.dtype:
            raise RuntimeError("linear_lora: out must be a contiguous [T, out] tensor of x's dtype")
        rc = _lib.check(self._lib.wp_linear_lora(self._handle, _ptr(y), _ptr(x2), _ptr(weight), int(weight.stride(0)),
                                                 _ptr(bias) if bias is not None else None, _ptr(wa_t_all),
                                                 int(wa_t_all.stride(0)), _ptr(wb_t_all), int(wb_t_all.stride(0)), L,
                                                 float(scale), rank, d_in, d_out, T, dt, self._stream()),
                        "linear_lora")
        return y if rc == _lib.WP_OK else None

    def add_lora_packed(self, y, x, wa_t_all, wb_t_all, scale, y_offset=None, y_slice_size=None) -> bool:
        """y += (scale * x . A[idx]^T) . B[idx]^T for the tokens of the last
        build_seg_bounds table (reference engine.py:56-62, bindings:195-234).
        Returns False (caller falls back) only for a rank without kernels."""
        off = int(y_offset or 0)
        return self.add_lora_slices(y, x, wa_t_all, [wb_t_all], scale, [off],
                                    [y_slice_size] if y_slice_size is not None else None)

    def add_lora_slices(self, y, x, wa_t_all, wb_t_alls: Sequence[torch.Tensor], scale,
                        y_offsets: Sequence[int], y_slice_sizes: Optional[Sequence[int]] = None) -> bool:
        """Several output slices in one launch: each wb_t_alls[i] ([L, 1, o_i, r])
        writes columns [y_offsets[i], y_offsets[i] + o_i) of y.  wa_t_all is one
        [L, 1, r, d] tensor shared by every slice (one shrink: packed q/k/v over
        one A) or a sequence with one per slice (vLLM's packed layers, each slice
        with its own lora_a); x is read once either way."""
        per_slice_a = isinstance(wa_t_all, (list, tuple))
        was = list(wa_t_all) if per_slice_a else [wa_t_all]
        rank = int(wb_t_alls[0].size(-1))
        ok = self._ranks.get(rank)
        if ok is None:
            ok = self._ranks[rank] = bool(self._ext.rank_supported(rank))
        if not ok:
            return False
        self._on_device(x, "x")
        self._on_device(y, "y")
        dt = _dtype_code(x, "x")
        if (y.dtype != x.dtype or any(w.dtype != x.dtype for w in was)
                or any(w.dtype != x.dtype for w in wb_t_alls)):
            raise RuntimeError("add_lora_packed: x, y and the LoRA weights must share one dtype")
        x2 = x.reshape(-1, x.size(-1))
        y2 = y.reshape(-1, y.size(-1))
        if not (x2.is_contiguous() and y2.is_contiguous()):
            raise RuntimeError("add_lora_packed: x/y must be contiguous")
        if y2.data_ptr() != y.data_ptr():
            raise RuntimeError("add_lora_packed: y must be viewable as 2-D in place")
        if not all(w.is_contiguous() for w in was) or not all(w.is_contiguous() for w in wb_t_alls):
            raise RuntimeError("add_lora_packed: wa_t_all/wb_t_all must be contiguous")
        T = int(x2.size(0))
        d_model = int(x2.size(1))
        L = int(was[0].size(0))
        n = len(wb_t_alls)
        if per_slice_a and len(was) != n:
            raise RuntimeError(f"add_lora_packed: {len(was)} lora_a tensors for {n} slices")
        for w in was:
            self._on_device(w, "wa_t_all")
            if int(w.size(0)) != L or int(w.size(-1)) != d_model or int(w.size(-2)) != rank:
                raise RuntimeError(f"add_lora_packed: wa_t_all {tuple(w.shape)} does not match x and rank {rank}")
        outs = []
        for i, w in enumerate(wb_t_alls):
            self._on_device(w, "wb_t_all")
            if int(w.size(0)) != L or int(w.size(-1)) != rank:
                raise RuntimeError(f"add_lora_packed: wb_t_all {tuple(w.shape)} does not match wa_t_all")
            o = int(w.size(-2))
            if y_slice_sizes is not None and y_slice_sizes[i] is not None and int(y_slice_sizes[i]) != o:
                raise RuntimeError(f"add_lora_packed: y_slice_size {y_slice_sizes[i]} != wb_t_all rows {o}")
            outs.append(o)
        if int(y2.size(0)) != T:
            raise RuntimeError("add_lora_packed: x and y have different token counts")
        wb_ptrs = (ctypes.c_void_p * n)(*[w.data_ptr() for w in wb_t_alls])
        wb_strides = (ctypes.c_int64 * n)(*[int(w.stride(0)) for w in wb_t_alls])
        o_arr = (ctypes.c_int32 * n)(*outs)
        off_arr = (ctypes.c_int32 * n)(*[int(v) for v in y_offsets])
        if per_slice_a:
            wa_ptrs = (ctypes.c_void_p * n)(*[w.data_ptr() for w in was])
            wa_strides = (ctypes.c_int64 * n)(*[int(w.stride(0)) for w in was])
            rc = _lib.check(self._lib.wp_add_lora_nslice(self._handle, _ptr(y2), _ptr(x2), n, wa_ptrs, wa_strides,
                                                         wb_ptrs, wb_strides, o_arr, off_arr, L, float(scale), rank,
                                                         d_model, T, int(y2.size(1)), dt, self._stream()),
                            "add_lora_packed_nslice")
        else:
            wa = was[0]
            rc = _lib.check(self._lib.wp_add_lora(self._handle, _ptr(y2), _ptr(x2), _ptr(wa), int(wa.stride(0)), L, n,
                                                  wb_ptrs, wb_strides, o_arr, off_arr, float(scale), rank, d_model, T,
                                                  int(y2.size(1)), dt, self._stream()),
                            "add_lora_packed")
        return rc == _lib.WP_OK

    def add_lora_packed_nslice(self, y, x, lora_a_stacked, lora_b_stacked, scale, output_slices) -> bool:
        """vLLM's PunicaWrapper.add_lora_packed_nslice shape: slice i has its own
        lora_a_stacked[i] [L, 1, r, d] and lora_b_stacked[i] [L, 1, o_i, r] and
        writes columns [sum(output_slices[:i]), + output_slices[i]) of y; every
        slice in one launch.  False (caller falls back) for a rank without
        kernels."""
        offs, acc = [], 0
        for o in output_slices:
            offs.append(acc)
            acc += int(o)
        return self.add_lora_slices(y, x, list(lora_a_stacked), list(lora_b_stacked), scale, offs,
                                    [int(o) for o in output_slices])

    # ------------------------------------------------- vLLM V1 LoRA ops --
    # The grouped ops behind vLLM V1's PunicaWrapperGPU (add_shrink,
    # add_expand, add_lora_embedding, add_lora_linear's bias), on the last
    # build_seg_bounds table; not in the reference, which hooks only the V0
    # add_lora (lora_warp_pipe/punica_wrapper.py:8-16).  Stacked weights as
    # vLLM holds them: lora_a [L, 1, r, d], lora_b [L, 1, o, r], bias
    # [L, 1, o] (or [L, o]).  Each returns False when the shapes have no
    # kernel (the caller falls back) and raises on invalid arguments.

    def _rank_ok(self, rank: int) -> bool:
        ok = self._ranks.get(rank)
        if ok is None:
            ok = self._ranks[rank] = bool(self._ext.rank_supported(rank))
        return ok

    def _stacked(self, ts: Sequence[torch.Tensor], dtype, what: str):
        for t in ts:
            self._on_device(t, what)
            if t.dtype != dtype:
                raise RuntimeError(f"{what} must have the activations' dtype {dtype}, got {t.dtype}")
            if t.dim() < 2 or not t[0].is_contiguous():
                raise RuntimeError(f"{what}: each adapter's matrix must be contiguous")
        n = len(ts)
        return ((ctypes.c_void_p * n)(*[t.data_ptr() for t in ts]),
                (ctypes.c_int64 * n)(*[int(t.stride(0)) for t in ts]))

    def lora_shrink(self, out: torch.Tensor, x: torch.Tensor, lora_a_stacked: Sequence[torch.Tensor],
                    scale: float) -> bool:
        """out[s][t, :r] += scale * x[t] . lora_a_stacked[s][id_t]^T in fp32,
        unrounded (V1's add_shrink / lora_shrink buffer); out is fp32
        [n_slices, T, >= r] (or a sequence of [T, >= r] views of one such
        tensor), 16-byte aligned with rows a multiple of 4 floats apart.
        Tokens without an adapter keep their rows."""
        was = list(lora_a_stacked)
        n = len(was)
        rank = int(was[0].size(-2))
        if n < 1 or n > 4 or not self._rank_ok(rank) or any(int(w.size(-2)) != rank for w in was):
            return False
        self._on_device(x, "x")
        dt = _dtype_code(x, "x")
        x2 = x.reshape(-1, x.size(-1))
        if not x2.is_contiguous():
            raise RuntimeError("lora_shrink: x must be contiguous")
        T, d = int(x2.size(0)), int(x2.size(1))
        L = int(was[0].size(0))
        if any(int(w.size(0)) != L or int(w.size(-1)) != d for w in was):
            raise RuntimeError("lora_shrink: every lora_a must be [L, 1, r, d] with x's d")
        a_ptrs, a_strides = self._stacked(was, x.dtype, "lora_a_stacked")
        outs = list(out) if isinstance(out, (list, tuple)) else [out[s] for s in range(int(out.size(0)))]
        if len(outs) != n:
            raise RuntimeError(f"lora_shrink: {len(outs)} output slices for {n} lora_a tensors")
        o0 = outs[0]
        for o in outs:
            self._on_device(o, "out")
            if o.dtype != torch.float32 or o.dim() != 2 or o.stride(1) != 1 or int(o.size(0)) < T:
                raise RuntimeError("lora_shrink: out slices must be fp32 [T, >= rank] with unit column stride")
            if o.stride(0) != o0.stride(0):
                raise RuntimeError("lora_shrink: out slices must share one row stride")
        row = int(o0.stride(0))
        sstride = (outs[1].data_ptr() - o0.data_ptr()) // 4 if n > 1 else 0
        if any(outs[s].data_ptr() != o0.data_ptr() + 4 * s * sstride for s in range(n)) or sstride < 0:
            raise RuntimeError("lora_shrink: out slices must be evenly spaced in one buffer")
        rc = _lib.check(self._lib.wp_lora_shrink(self._handle, _ptr(o0), sstride, row, _ptr(x2), n, a_ptrs, a_strides, L,
                                                 float(scale), rank, d, T, dt, self._stream()), "lora_shrink")
        return rc == _lib.WP_OK

    def _bias_args(self, biases, y, n: int, what: str):
        bs = list(biases) if biases is not None else [None] * n
        if len(bs) != n:
            raise RuntimeError(f"{what}: {len(bs)} biases for {n} slices")
        ptrs, strides = [], []
        for b in bs:
            if b is None:
                ptrs.append(None)
                strides.append(0)
                continue
            self._on_device(b, "lora_bias_stacked")
            if b.dtype != y.dtype:
                raise RuntimeError(f"{what}: lora_bias_stacked must have y's dtype")
            b2 = b.reshape(b.size(0), -1)
            if b2.stride(1) != 1 or b2.data_ptr() != b.data_ptr():
                raise RuntimeError(f"{what}: each adapter's bias row must be contiguous")
            ptrs.append(b.data_ptr())
            strides.append(int(b2.stride(0)))
        return (ctypes.c_void_p * n)(*ptrs), (ctypes.c_int64 * n)(*strides), any(b is not None for b in bs)

    def add_bias(self, y: torch.Tensor, lora_bias_stacked, output_slices: Sequence[int], num_loras: int,
                 offset_start: int = 0) -> None:
        """V1's _apply_bias: y[t, window s] = rn(y[t, window s] + bias[s][id_t])
        for every token with an adapter and every slice whose bias is not
        None; slice windows are consecutive from offset_start."""
        self._on_device(y, "y")
        dt = _dtype_code(y, "y")
        y2 = y.reshape(-1, y.size(-1))
        if not y2.is_contiguous() or y2.data_ptr() != y.data_ptr():
            raise RuntimeError("add_bias: y must be contiguous")
        n = len(output_slices)
        offs = [int(offset_start) + sum(int(o) for o in output_slices[:i]) for i in range(n)]
        b_ptrs, b_strides, _ = self._bias_args(lora_bias_stacked, y, n, "add_bias")
        o_arr = (ctypes.c_int32 * n)(*[int(o) for o in output_slices])
        off_arr = (ctypes.c_int32 * n)(*offs)
        _lib.check(self._lib.wp_add_bias(self._handle, _ptr(y2), int(y2.size(1)), n, b_ptrs, b_strides, o_arr, off_arr,
                                         int(num_loras), int(y2.size(0)), dt, self._stream()), "add_bias")

    def lora_expand(self, y: torch.Tensor, h: torch.Tensor, lora_b_stacked: Sequence[torch.Tensor],
                    output_slices: Sequence[int], offset_start: int = 0, add_inputs: bool = True,
                    lora_bias_stacked=None) -> bool:
        """V1's lora_expand: for every slice s and token t with an adapter,
        y[t, off_s + o] = rn((add_inputs ? y'[t, off_s + o] : 0) + rn(h[s][t]) . B_s[id_t][o]^T)
        with slice windows consecutive from offset_start and y' = rn(y + bias)
        where lora_bias_stacked[s] is given (add_inputs only).  h: [n, T, r]
        fp32 (rounded to y's dtype first, as V1 casts it) or y's dtype.  Two
        launches; tokens without an adapter keep their rows."""
        wbs = list(lora_b_stacked)
        n = len(wbs)
        rank = int(wbs[0].size(-1))
        if n < 1 or n > 4 or not self._rank_ok(rank) or any(int(w.size(-1)) != rank for w in wbs):
            return False
        self._on_device(y, "y")
        self._on_device(h, "h")
        dt = _dtype_code(y, "y")
        y2 = y.reshape(-1, y.size(-1))
        if not y2.is_contiguous() or y2.data_ptr() != y.data_ptr():
            raise RuntimeError("lora_expand: y must be contiguous")
        T = int(y2.size(0))
        if h.dim() != 3 or int(h.size(0)) != n or h.stride(2) != 1 or int(h.size(1)) < T or int(h.size(2)) < rank:
            raise RuntimeError(f"lora_expand: h must be [{n}, >= {T}, >= {rank}] with unit column stride")
        if h.dtype not in (torch.float32, y.dtype):
            raise RuntimeError("lora_expand: h must be fp32 or y's dtype")
        L = int(wbs[0].size(0))
        outs = [int(o) for o in output_slices]
        if len(outs) != n or any(int(w.size(0)) != L or int(w.size(-2)) != o for w, o in zip(wbs, outs)):
            raise RuntimeError("lora_expand: lora_b_stacked[s] must be [L, 1, output_slices[s], r]")
        b_ptrs, b_strides = self._stacked(wbs, y.dtype, "lora_b_stacked")
        bias_ptrs, bias_strides, _ = self._bias_args(lora_bias_stacked, y, n, "lora_expand")
        offs = [int(offset_start) + sum(outs[:i]) for i in range(n)]
        o_arr = (ctypes.c_int32 * n)(*outs)
        off_arr = (ctypes.c_int32 * n)(*offs)
        rc = _lib.check(self._lib.wp_lora_expand(self._handle, _ptr(y2), int(y2.size(1)), _ptr(h),
                                                 1 if h.dtype == torch.float32 else 0, int(h.stride(0)),
                                                 int(h.stride(1)), n, b_ptrs, b_strides, o_arr, off_arr, bias_ptrs,
                                                 bias_strides, L, rank, T, 1 if add_inputs else 0, dt, self._stream()),
                        "lora_expand")
        return rc == _lib.WP_OK

    # ------------------------------------------------------------- staging --
    def prefetch_adapter(self, adapter_id, layer=None) -> int:
        """Stages the adapter's A/B in a slot on the prefetch stream; returns the
        slot index or -1 (unknown id / pool exhausted) (reference bindings:46-57)."""
        slot = ctypes.c_int32(-1)
        _lib.check(self._lib.wp_prefetch_adapter(self._handle, self._store_id(adapter_id, layer), ctypes.byref(slot)),
                   "prefetch_adapter")
        return int(slot.value)

    def prefetch_adapters(self, adapter_ids, layer=None) -> List[int]:
        """prefetch_adapter for several ids in one call (one copy kernel);
        returns their slots (-1 where none)."""
        ids = [self._store_id(a, layer) for a in adapter_ids]
        n = len(ids)
        arr = (ctypes.c_int32 * max(n, 1))(*ids)
        out = (ctypes.c_int32 * max(n, 1))()
        _lib.check(self._lib.wp_prefetch_adapters(self._handle, arr, n, out), "prefetch_adapters")
        return [int(out[k]) for k in range(n)]

    def release_prefetches(self, adapter_ids, layer=None) -> None:
        """release_prefetch for several ids in one call (one launch)."""
        ids = [self._store_id(a, layer) for a in adapter_ids]
        arr = (ctypes.c_int32 * max(len(ids), 1))(*ids)
        _lib.check(self._lib.wp_release_prefetches(self._handle, arr, len(ids), self._stream()), "release_prefetch")

    def wait_prefetches(self, adapter_ids, layer=None) -> bool:
        """wait_prefetch for several ids in one call; False if any holds no slot."""
        ids = [self._store_id(a, layer) for a in adapter_ids]
        arr = (ctypes.c_int32 * max(len(ids), 1))(*ids)
        rc = _lib.check(self._lib.wp_wait_prefetches(self._handle, arr, len(ids), self._stream()), "wait_prefetch")
        return rc == _lib.WP_OK

    def is_prefetch_ready(self, adapter_id, layer=None) -> bool:
        r = ctypes.c_int32(0)
        _lib.check(self._lib.wp_is_prefetch_ready(self._handle, self._store_id(adapter_id, layer), ctypes.byref(r)),
                   "is_prefetch_ready")
        return bool(r.value)

    def release_prefetch(self, adapter_id, layer=None):
        """Frees the id's slot in stream order on torch's current stream: work
        already enqueued there (graph replays included) still reads the slot,
        work enqueued after it does not, and the slot's next copy waits for
        that point (reference bindings:64 frees it at once)."""
        _lib.check(self._lib.wp_release_prefetch(self._handle, self._store_id(adapter_id, layer), self._stream()),
                   "release_prefetch")

    def wait_prefetch(self, adapter_id, layer=None) -> bool:
        """Makes torch's current stream wait (on the device) until the id's
        prefetch copy has landed; False when the id holds no slot.  A
        build_seg_bounds enqueued after it (captured or not) uses the staged
        copy."""
        rc = _lib.check(self._lib.wp_wait_prefetch(self._handle, self._store_id(adapter_id, layer), self._stream()),
                        "wait_prefetch")
        return rc == _lib.WP_OK

    def set_spin_limit(self, polls: Optional[int] = None) -> None:
        """Test and debug: polls before a wait on partials gives up (None: the
        default, about 0.1 s).  After a give-up (device error 8), calls that use
        the partial buffer skip their work until the next plan build repairs it."""
        _lib.check(self._lib.wp_set_spin_limit(self._handle, 0xFFFFFFFF if polls is None else int(polls)),
                   "set_spin_limit")
