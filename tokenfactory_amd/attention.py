"""``slot_based_attention``: the reference's ``_slot_based_attention`` on gfx950 kernels.

Same inputs, output and branch semantics as
``Qwen3_8FullAttention._slot_based_attention`` (reference
``qwen3_8/full_attention.py:163-283``):

* ``bsz == 1``: context length from ``batch.max_seq_len`` (``:186``); causal
  mask only when ``ext_len > 1`` (``:200-208``);
* pure decode (``max_extend_len == 1``): one query per request, keys
  ``k < seq_lens[b]`` (``:231-242``) -> ``tf_attn_decode`` over the whole batch,
  no host metadata at all;
* extend / mixed: query ``t`` of request ``b`` sees keys
  ``k <= seq_lens[b] - ext_b + t`` (``:266-278``) -> ``tf_attn_extend`` over
  the requests with ``ext_b > 1`` plus ``tf_attn_decode`` over the ``ext_b == 1``
  rows of a mixed batch; the two work lists are planned on the host from
  ``batch.extend_lens`` and uploaded in one copy.

``SlotAttentionCall`` separates planning (argument checks, work lists, upload,
workspace) from launching, so a step's launches can be repeated or timed phase
by phase. Only ROCm device tensors are accepted; there is no CPU path.
"""
from __future__ import annotations

import threading
from typing import Dict, Optional, Tuple

import numpy as np
import torch

from . import _native
from .planning import plan_decode_items, plan_extend

_KV_DTYPES = {
    torch.bfloat16: _native.TF_DTYPE_BF16,
    torch.float8_e4m3fn: _native.TF_DTYPE_FP8_E4M3,
}

_ws_lock = threading.Lock()
_workspaces: Dict[Tuple[int, int], torch.Tensor] = {}


def _workspace(device: torch.device, stream: torch.cuda.Stream, nbytes: int) -> torch.Tensor:
    """Decode split-partial scratch, one per (device, stream), grown on demand."""
    key = (device.index if device.index is not None else torch.cuda.current_device(),
           stream.cuda_stream)
    with _ws_lock:
        ws = _workspaces.get(key)
        if ws is None or ws.numel() < nbytes:
            ws = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
            _workspaces[key] = ws
        return ws


class _Uploader:
    """Host -> device copies of per-step plan lists through a ring of pinned
    staging buffers (allocated once, grown on demand), so that a step neither
    allocates pinned memory nor copies from pageable memory, either of which
    can block the host until the GPU has caught up.  A slot is reused only
    after its previous copy has executed (its event)."""

    SLOTS = 32

    def __init__(self):
        self.bufs = [None] * self.SLOTS
        self.events = [None] * self.SLOTS
        self.next = 0

    def upload(self, arr: np.ndarray, device: torch.device,
               stream: torch.cuda.Stream) -> torch.Tensor:
        i = self.next
        self.next = (i + 1) % self.SLOTS
        ev = self.events[i]
        if ev is not None:
            ev.synchronize()
        buf = self.bufs[i]
        if buf is None or buf.numel() < arr.size:
            buf = torch.empty(max(arr.size, 1 << 16), dtype=torch.int32, pin_memory=True)
            self.bufs[i] = buf
        buf[: arr.size].numpy()[:] = arr
        with torch.cuda.stream(stream):
            dev = torch.empty(arr.size, dtype=torch.int32, device=device)
            dev.copy_(buf[: arr.size], non_blocking=True)
        if ev is None:
            ev = torch.cuda.Event()
            self.events[i] = ev
        ev.record(stream)
        return dev


_uploaders: Dict[int, _Uploader] = {}


def _upload(arr: np.ndarray, device: torch.device, stream: torch.cuda.Stream) -> torch.Tensor:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    with _ws_lock:
        up = _uploaders.get(idx)
        if up is None:
            up = _Uploader()
            _uploaders[idx] = up
        return up.upload(arr, device, stream)


_fork_events: Dict[Tuple[int, int], Tuple[torch.cuda.Event, torch.cuda.Event]] = {}


def _fork_join_events(device: torch.device, main: torch.cuda.Stream):
    """Two events per (device, caller stream), created once and re-recorded by
    every mixed step on that stream (a wait enqueued earlier keeps the record
    it saw).  Events made per step and destroyed while their waits are still
    queued stall the host by about a step on ROCm."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    key = (idx, main.cuda_stream)
    with _ws_lock:
        ev = _fork_events.get(key)
        if ev is None:
            ev = (torch.cuda.Event(), torch.cuda.Event())
            _fork_events[key] = ev
        return ev


_cu_counts: Dict[int, int] = {}


def _cu_count(device: torch.device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    n = _cu_counts.get(idx)
    if n is None:
        n = _cu_counts[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return n


_side_streams: Dict[int, torch.cuda.Stream] = {}


def _side_stream(device: torch.device) -> torch.cuda.Stream:
    """A second stream per device (default priority) for the decode launches of
    a mixed step, which then run beside the extend kernel."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    with _ws_lock:
        st = _side_streams.get(idx)
        if st is None:
            st = torch.cuda.Stream(device=idx)
            _side_streams[idx] = st
        return st


_plan_events: Dict[Tuple[int, int], torch.cuda.Event] = {}


def _plan_event(device: torch.device, stream: torch.cuda.Stream) -> torch.cuda.Event:
    """One reusable event per (device, planning stream), recorded behind a
    shared step plan for the other streams that read it."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    key = (idx, stream.cuda_stream)
    ev = _plan_events.get(key)
    if ev is None:
        ev = torch.cuda.Event()
        _plan_events[key] = ev
    return ev


class StepPlan:
    """The work lists of one model step for one head layout: the extend work
    entries and the decode items / rows of a ``ForwardBatch``, planned on the
    device (``tf_attn_plan_device``, from ``extend_lens_tensor``) by the first
    attention call of the step and read by every later one.

    A model step runs every full-attention layer over the same batch
    (``decoder_layer.py:68-69`` calls the attention once per layer), so the
    lists do not change between layers; ``slot_based_attention`` keeps one
    ``StepPlan`` per (device, T, q heads, kv heads) on the batch object itself.
    Calls on another stream than the planning one wait for the plan (an event
    recorded on the planning stream)."""

    def __init__(self, batch, n_tok: int, n_q: int, n_kv: int, device: torch.device):
        bsz = batch.batch_size
        ext_t = batch.extend_lens_tensor
        if ext_t is None or ext_t.device != device or ext_t.dtype != torch.long \
                or ext_t.numel() != bsz or not ext_t.is_contiguous():
            raise ValueError("a device plan needs batch.extend_lens_tensor: contiguous int64 "
                             "[batch_size] on q's device")
        self.batch_size, self.n_q, self.n_kv = bsz, n_q, n_kv
        self.ext_t = ext_t
        self.n_work = _native.plan_device_capacity(n_tok, bsz, n_q, n_kv)
        self.n_dec = bsz
        self.meta = torch.empty(self.n_work * 8 + 2 * bsz + 4, dtype=torch.int32, device=device)
        base = self.meta.data_ptr() + 4 * self.n_work * 8
        self.items = _DevPtr(base)
        self.rows = _DevPtr(base + 4 * bsz)
        self.status = _DevPtr(base + 8 * bsz)
        self.device = device
        self._lock = threading.Lock()
        self._planned_on: Optional[torch.cuda.Stream] = None
        self._event: Optional[torch.cuda.Event] = None

    def ensure(self, stream: torch.cuda.Stream) -> None:
        """Plan on ``stream`` if no call has yet; else order ``stream`` after
        the plan."""
        with self._lock:
            if self._planned_on is None:
                _native.call("tf_attn_plan_device", self.ext_t.data_ptr(), self.batch_size,
                             self.n_q, self.n_kv, 1, self.meta.data_ptr(), self.n_work,
                             self.items.data_ptr(), self.rows.data_ptr(), self.n_dec,
                             self.status.data_ptr(), stream.cuda_stream)
                with _ws_lock:
                    self._event = _plan_event(self.device, stream)
                    self._event.record(stream)
                self._planned_on = stream
            elif self._planned_on.cuda_stream != stream.cuda_stream:
                # (a later step planned on the same stream may have recorded the
                # event again: the wait then covers more than this plan)
                stream.wait_event(self._event)


_STEP_PLANS = "_tf_attn_step_plans"


def step_plan(batch, n_tok: int, n_q: int, n_kv: int, device: torch.device) -> StepPlan:
    """The ``StepPlan`` of ``batch`` for this head layout (made on first use)."""
    key = (device.index, n_tok, n_q, n_kv)
    with _ws_lock:
        plans = getattr(batch, _STEP_PLANS, None)
        if plans is None:
            plans = {}
            setattr(batch, _STEP_PLANS, plans)
        plan = plans.get(key)
        if plan is None:
            plan = StepPlan(batch, n_tok, n_q, n_kv, device)
            plans[key] = plan
        return plan


def _ptr(t) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _require_device(name: str, t: torch.Tensor, device: torch.device) -> None:
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")


def _check_inputs(q, k_buf, v_buf, batch):
    if not q.is_cuda:
        raise RuntimeError(
            "slot_based_attention runs only on ROCm devices (q is on "
            f"{q.device}); there is no CPU implementation")
    if q.dim() != 3 or k_buf.dim() != 3 or v_buf.shape != k_buf.shape:
        raise ValueError(f"expected q [T,Hq,D] and pools [S,Hkv,D], got {tuple(q.shape)}, "
                         f"{tuple(k_buf.shape)}, {tuple(v_buf.shape)}")
    if q.dtype != torch.bfloat16:
        raise NotImplementedError(f"q dtype {q.dtype} (bf16 only)")
    if k_buf.dtype not in _KV_DTYPES or v_buf.dtype != k_buf.dtype:
        raise NotImplementedError(f"KV pool dtype {k_buf.dtype}")
    if q.shape[2] != k_buf.shape[2]:
        raise ValueError("q and pool head_dim differ")
    if not (k_buf.is_contiguous() and v_buf.is_contiguous()):
        raise ValueError("KV pools must be contiguous [S, Hkv, D] layer views")
    dev = q.device
    for name, t in (("layer_k_buffer", k_buf), ("layer_v_buffer", v_buf),
                    ("req_to_token", batch.req_to_token),
                    ("req_pool_indices", batch.req_pool_indices),
                    ("seq_lens", batch.seq_lens)):
        _require_device(name, t, dev)
    rtt = batch.req_to_token
    if rtt.dtype != torch.int64 or rtt.dim() != 2 or rtt.stride(1) != 1:
        raise ValueError("req_to_token must be a row-major int64 [max_reqs, max_ctx] tensor")
    if batch.req_pool_indices.dtype != torch.int64 or batch.seq_lens.dtype != torch.int64:
        raise ValueError("req_pool_indices / seq_lens must be int64")
    if not (batch.req_pool_indices.is_contiguous() and batch.seq_lens.is_contiguous()):
        raise ValueError("req_pool_indices / seq_lens must be contiguous")
    if batch.max_seq_len > rtt.shape[1]:
        raise ValueError(f"max_seq_len {batch.max_seq_len} exceeds req_to_token width "
                         f"{rtt.shape[1]}")


class _DevPtr:
    """A raw device address posing as a tensor for ``_ptr``."""

    __slots__ = ("_addr",)

    def __init__(self, addr: int):
        self._addr = addr

    def data_ptr(self) -> int:
        return self._addr


class SlotAttentionCall:
    """One planned ``_slot_based_attention`` step: validated arguments, uploaded
    work lists and workspace, ready to launch (repeatedly) on ``stream``.

    ``run()`` enqueues every kernel of the step. For timing, ``run_extend()``,
    ``run_decode_partial()`` and ``run_decode_merge()`` enqueue the individual
    launches; run in that order they are exactly ``run()``.

    ``overlap_decode`` (default: ``device_plan``): on a mixed step, run the
    decode launches on a second stream beside the extend kernel (the results
    are identical).  The fork / join events are cached per (device, stream),
    so calls made per step do not create events (events destroyed while
    their waits are still queued stall the host on ROCm).

    ``step_plan``: the batch's shared ``StepPlan`` (implies the device plan);
    ``run()`` then plans only if no earlier call of the step did.

    ``out_amax`` (optional 1-element int32 tensor on q's device): every launch
    raises it to the largest bf16 bit pattern of ``|out|`` it writes (sign
    cleared, so it orders like the floats and NaN sorts above inf), the amax
    of the FP8 quantisation in front of ``o_proj``
    (``quantize_activations(..., amax=out_amax)``); the caller zeroes it before
    ``run()``.
    """

    def __init__(self, q, layer_k_buffer, layer_v_buffer, batch, *, scaling=None,
                 k_scale=None, v_scale=None, decode_workgroups: int = 0, out=None,
                 stream=None, gate=None, device_plan: bool = False,
                 overlap_decode: Optional[bool] = None, out_amax=None,
                 step_plan: Optional[StepPlan] = None):
        _check_inputs(q, layer_k_buffer, layer_v_buffer, batch)
        n_tok, n_q, head_dim = q.shape
        n_slots, n_kv, _ = layer_k_buffer.shape
        if n_q % n_kv:
            raise ValueError(f"num_q_heads {n_q} is not a multiple of num_kv_heads {n_kv}")
        if scaling is None:
            scaling = head_dim ** -0.5
        kv_dtype = _KV_DTYPES[layer_k_buffer.dtype]
        if kv_dtype == _native.TF_DTYPE_FP8_E4M3:
            if k_scale is None or v_scale is None:
                raise ValueError("an fp8 KV pool needs k_scale and v_scale")
            k_scale = k_scale.to(device=q.device, dtype=torch.float32).reshape(1).contiguous()
            v_scale = v_scale.to(device=q.device, dtype=torch.float32).reshape(1).contiguous()
        else:
            k_scale = v_scale = None
        if q.stride(2) != 1 or q.stride(1) != head_dim:
            q = q.contiguous()
        if out is None:
            out = torch.empty((n_tok, n_q, head_dim), dtype=q.dtype, device=q.device)
        elif out.shape != q.shape or out.dtype != q.dtype or out.stride(2) != 1 \
                or out.stride(1) != head_dim:
            raise ValueError("out must match q's shape/dtype with dense heads and dims")

        if gate is not None:
            if gate.shape != q.shape or gate.dtype != torch.bfloat16 or gate.device != q.device \
                    or gate.stride(2) != 1 or gate.stride(0) % 8 or gate.stride(1) % 8 \
                    or gate.data_ptr() % 16:
                raise ValueError("gate must be a bf16 [T, Hq, D] view on q's device with "
                                 "contiguous dims, strides in multiples of 8 and a 16-byte "
                                 "aligned start")
            self._epilogue_args = (gate.data_ptr(), gate.stride(0), gate.stride(1))
        else:
            self._epilogue_args = (None, 0, 0)
        self.gate = gate
        if out_amax is not None and (out_amax.dtype != torch.int32 or out_amax.numel() != 1
                                     or out_amax.device != q.device):
            raise ValueError("out_amax must be a 1-element int32 tensor on q's device")
        self.out_amax = out_amax
        # the launches' trailing arguments: gate, its strides, out_amax
        self._epilogue_args = self._epilogue_args + (_ptr(out_amax),)

        bsz = batch.batch_size
        ext_lens = [int(e) for e in batch.extend_lens]
        if len(ext_lens) != bsz or sum(ext_lens) != n_tok:
            raise ValueError(f"extend_lens {ext_lens[:8]}... do not match batch_size={bsz}, "
                             f"T={n_tok}")
        self.q, self.out = q, out
        self.k_buf, self.v_buf = layer_k_buffer, layer_v_buffer
        self.k_scale, self.v_scale = k_scale, v_scale
        self.batch = batch
        self._fixed_stream = stream
        self._shared_plan = step_plan
        self.device_plan = bool(device_plan) or step_plan is not None
        self.n_q, self.n_kv, self.head_dim = n_q, n_kv, head_dim
        self.scaling = float(scaling)
        self.decode_workgroups = int(decode_workgroups)
        self.max_len = int(batch.max_seq_len)
        rtt = batch.req_to_token
        seq_override = self.max_len if bsz == 1 else 0
        self._pool_args = (layer_k_buffer.data_ptr(), layer_v_buffer.data_ptr(), n_slots,
                           kv_dtype, _ptr(k_scale), _ptr(v_scale),
                           rtt.data_ptr(), rtt.shape[0], rtt.stride(0), rtt.shape[1],
                           batch.req_pool_indices.data_ptr(), batch.seq_lens.data_ptr(),
                           seq_override)
        self.overlap_decode = (self.device_plan if overlap_decode is None
                               else bool(overlap_decode))
        self.n_work = 0
        self.n_dec = 0
        self._meta = None
        self._items = self._rows = None
        self._status = None
        if n_tok == 0:
            return
        if step_plan is not None:
            if (step_plan.batch_size, step_plan.n_q, step_plan.n_kv) != (bsz, n_q, n_kv) \
                    or step_plan.device != q.device:
                raise ValueError("step_plan was made for another batch layout or device")
            self.n_work, self.n_dec = step_plan.n_work, step_plan.n_dec
            self._ext_t = step_plan.ext_t
            self._meta = step_plan.meta
            self._items, self._rows, self._status = (step_plan.items, step_plan.rows,
                                                     step_plan.status)
        elif self.device_plan:
            # Lists built on the device at every run() from extend_lens_tensor,
            # padded to capacities fixed by T and B (graph-capturable step).
            ext_t = batch.extend_lens_tensor
            if ext_t is None or ext_t.device != q.device or ext_t.dtype != torch.long \
                    or ext_t.numel() != bsz or not ext_t.is_contiguous():
                raise ValueError("device_plan needs batch.extend_lens_tensor: contiguous int64 "
                                 "[batch_size] on q's device")
            self.n_work = _native.plan_device_capacity(n_tok, bsz, n_q, n_kv)
            self.n_dec = bsz
            self._ext_t = ext_t
            self._meta = torch.empty(self.n_work * 8 + 2 * bsz + 4, dtype=torch.int32,
                                     device=q.device)
            base = self._meta.data_ptr() + 4 * self.n_work * 8
            self._items = _DevPtr(base)
            self._rows = _DevPtr(base + 4 * bsz)
            self._status = _DevPtr(base + 8 * bsz)
        elif batch.max_extend_len == 1 or (bsz == 1 and ext_lens[0] == 1):
            # Pure decode: batch entry b is query row b; nothing to upload.
            self.n_dec = bsz
        else:
            if torch.cuda.is_current_stream_capturing():
                # The host plan reaches the device through a reused pinned
                # staging slot: a captured copy would replay stale plans.
                raise RuntimeError("a host-planned extend step cannot be captured in a graph; "
                                   "build the call with device_plan=True")
            work = plan_extend(ext_lens, n_q, n_kv, decode_to_decode_kernel=True)
            items, rows = plan_decode_items(ext_lens)
            self.n_work, self.n_dec = len(work), len(items)
            meta = np.zeros(self.n_work * 8 + 2 * self.n_dec + 4, dtype=np.int32)
            meta[: self.n_work * 8] = work.reshape(-1)
            meta[self.n_work * 8: self.n_work * 8 + self.n_dec] = items
            meta[self.n_work * 8 + self.n_dec: self.n_work * 8 + 2 * self.n_dec] = rows
            self._meta = _upload(meta, q.device, self.stream)
            base = self._meta.data_ptr() + 4 * self.n_work * 8
            if self.n_dec:
                self._items = _DevPtr(base)
                self._rows = _DevPtr(base + 4 * self.n_dec)
        if (self.decode_workgroups == 0 and self.n_work and self.n_dec
                and max(ext_lens) > 1 and min(ext_lens) == 1):
            # A mixed step's decode kernel runs beside the extend kernel, whose
            # workgroups hold whole CUs: three times as many, shorter decode
            # workgroups fill the CUs the extend kernel frees as it drains
            # (mixed step 1350 -> 1310 us per layer).  The rule depends on the
            # batch alone, so a serial call gives the same bits.
            self.decode_workgroups = 3 * _cu_count(q.device)
        self.ws = None
        if self.n_dec:
            nbytes = _native.decode_workspace_bytes(self.n_dec, n_q, n_kv, head_dim,
                                                    self.max_len, self.decode_workgroups)
            if nbytes:
                self.ws = _workspace(q.device, self.stream, nbytes)

    @property
    def stream(self) -> torch.cuda.Stream:
        """The stream given at construction, else the current one at launch time
        (so a call built outside a graph capture launches into the capture)."""
        if self._fixed_stream is not None:
            return self._fixed_stream
        return torch.cuda.current_stream(self.q.device)

    # -- launches
    def run_plan(self) -> None:
        """Device-side planning (device_plan=True): the work and decode lists
        (with a shared step plan: only if no earlier call of the step planned)."""
        if self._shared_plan is not None:
            if self.n_work:
                self._shared_plan.ensure(self.stream)
            return
        if self.device_plan and self.n_work:
            base = self._meta.data_ptr()
            _native.call("tf_attn_plan_device", self._ext_t.data_ptr(), self.batch.batch_size,
                         self.n_q, self.n_kv, 1, base, self.n_work, self._items.data_ptr(),
                         self._rows.data_ptr(), self.n_dec, self._status.data_ptr(),
                         self.stream.cuda_stream)

    def plan_status(self):
        """(real work entries, real decode items, flags) of the last device plan:
        flags bit 0 = capacity exceeded, bit 1 = an extend length outside [1, 2^31)."""
        if self._status is None:
            return None
        n = self.n_work * 8 + 2 * self.n_dec
        return tuple(int(x) for x in self._meta[n:n + 3].cpu())

    def _decode(self, entry: str, stream: Optional[torch.cuda.Stream] = None) -> None:
        if not self.n_dec:
            return
        ws = self.ws
        stream = stream if stream is not None else self.stream
        _native.call(entry, self.q.data_ptr(), self.q.stride(0), *self._pool_args,
                     _ptr(self._items), _ptr(self._rows), self.n_dec,
                     self.n_q, self.n_kv, self.head_dim, self.scaling,
                     self.out.data_ptr(), self.out.stride(0),
                     _ptr(ws), 0 if ws is None else ws.numel(), self.max_len,
                     self.decode_workgroups, *self._epilogue_args, stream.cuda_stream)

    def run_extend(self) -> None:
        if self.n_work:
            _native.call("tf_attn_extend", self.q.data_ptr(), self.q.stride(0),
                         *self._pool_args, self._meta.data_ptr(), self.n_work,
                         self.n_q, self.n_kv, self.head_dim, self.scaling,
                         self.out.data_ptr(), self.out.stride(0), *self._epilogue_args,
                         self.stream.cuda_stream)

    def run_decode_partial(self) -> None:
        self._decode("tf_attn_decode_partial")

    def run_decode_merge(self) -> None:
        self._decode("tf_attn_decode_merge")

    def run(self) -> torch.Tensor:
        self.run_plan()
        if self.n_work and self.n_dec and self.overlap_decode:
            # Mixed step: the HBM-bound decode launches go to a second stream and
            # run beside the MFMA-bound extend kernel (they write disjoint rows
            # of out); the caller's stream waits for both.
            # The extend launch goes out first (the decode launch waits only
            # for the work before it): neither kernel's workgroup fits beside
            # the other's on a CU, so the decode workgroups take the CUs the
            # extend kernel's last round leaves idle, rather than the extend
            # kernel waiting for the decode kernel's persistent grid.
            main, side = self.stream, _side_stream(self.q.device)
            fork, join = _fork_join_events(self.q.device, main)
            fork.record(main)
            self.run_extend()
            side.wait_event(fork)
            self._decode("tf_attn_decode", side)
            join.record(side)
            main.wait_event(join)
        else:
            self.run_extend()
            self._decode("tf_attn_decode")
        return self.out


def slot_based_attention(
    q: torch.Tensor,
    layer_k_buffer: torch.Tensor,
    layer_v_buffer: torch.Tensor,
    batch,
    *,
    scaling: Optional[float] = None,
    k_scale: Optional[torch.Tensor] = None,
    v_scale: Optional[torch.Tensor] = None,
    decode_workgroups: int = 0,
    out: Optional[torch.Tensor] = None,
    gate: Optional[torch.Tensor] = None,
    out_amax: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Attention of ``q [T, Hq, D]`` over one layer's slot pool; returns ``[T, Hq, D]``.

    A step with extend work is planned once: the first call made with a
    ``ForwardBatch`` plans its work lists on the device and keeps them on the
    batch (``StepPlan``); the calls of the step's other layers reuse them.  A
    call under graph capture plans inside the graph instead.  On a mixed step
    the decode launches run on a second stream beside the extend kernel
    (identical results).

    ``scaling`` defaults to ``head_dim ** -0.5`` (``full_attention.py:40``).
    ``k_scale`` / ``v_scale`` (fp32 device scalars) are required for a
    ``float8_e4m3fn`` pool. ``decode_workgroups`` overrides the size of the
    decode kernel's persistent grid (0 = one workgroup per compute unit, three
    per compute unit on a step that mixes extends and decodes).
    ``gate`` (bf16 ``[T, Hq, D]``, any view with contiguous dims): the result is
    ``attn * F.silu(gate)`` (``full_attention.py:157-159``), computed in the
    kernels' output write with the same bf16 roundings. ``out_amax``: see
    ``SlotAttentionCall``.
    """
    plan, device_plan = None, False
    if q.is_cuda and q.dim() == 3 and q.shape[0] and layer_k_buffer.dim() == 3 \
            and _plannable(batch, q.device):
        if torch.cuda.is_current_stream_capturing():
            # A captured call plans inside the graph (its plan runs at every
            # replay) and shares nothing with eager calls of the batch.
            device_plan = True
        else:
            plan = step_plan(batch, q.shape[0], q.shape[1], layer_k_buffer.shape[1], q.device)
    call = SlotAttentionCall(q, layer_k_buffer, layer_v_buffer, batch, scaling=scaling,
                             k_scale=k_scale, v_scale=v_scale,
                             decode_workgroups=decode_workgroups, out=out, gate=gate,
                             out_amax=out_amax, step_plan=plan, device_plan=device_plan)
    return call.run()


def _plannable(batch, device: torch.device) -> bool:
    """Whether the step has extend work and the batch carries the device copy
    of its extend lengths (pure decode steps need no plan at all)."""
    if batch.max_extend_len <= 1 or (batch.batch_size == 1 and int(batch.extend_lens[0]) == 1):
        return False
    ext_t = batch.extend_lens_tensor
    return (ext_t is not None and ext_t.device == device and ext_t.dtype == torch.long
            and ext_t.numel() == batch.batch_size and ext_t.is_contiguous())


def gather_kv(pool: torch.Tensor, req_to_token: torch.Tensor, req_pool_indices: torch.Tensor,
              max_len: int) -> torch.Tensor:
    """``pool[req_to_token[req_pool_indices, :max_len].clamp(min=0)]`` via ``tf_gather_kv``."""
    if not pool.is_cuda:
        raise RuntimeError("gather_kv runs only on ROCm devices")
    dtype_code = {torch.bfloat16: _native.TF_DTYPE_BF16,
                  torch.float8_e4m3fn: _native.TF_DTYPE_FP8_E4M3,
                  torch.float32: _native.TF_DTYPE_FP32}[pool.dtype]
    if not pool.is_contiguous():
        raise ValueError("pool must be contiguous")
    if req_to_token.stride(1) != 1 or req_to_token.dtype != torch.int64:
        raise ValueError("req_to_token must be row-major int64")
    bsz = req_pool_indices.numel()
    rpi = req_pool_indices.to(torch.int64).contiguous()
    row_elems = int(np.prod(pool.shape[1:]))
    out = torch.empty((bsz, max_len, *pool.shape[1:]), dtype=pool.dtype, device=pool.device)
    _native.call("tf_gather_kv", pool.data_ptr(), dtype_code, pool.shape[0], row_elems,
                 req_to_token.data_ptr(), req_to_token.shape[0], req_to_token.stride(0),
                 req_to_token.shape[1], rpi.data_ptr(), bsz, max_len,
                 out.data_ptr(), torch.cuda.current_stream(pool.device).cuda_stream)
    return out


def write_kv(layer_k_buffer: torch.Tensor, layer_v_buffer: torch.Tensor,
             out_cache_loc: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
             k_scale: Optional[torch.Tensor] = None,
             v_scale: Optional[torch.Tensor] = None) -> None:
    """``layer_k_buffer[out_cache_loc] = k`` (and v) via ``tf_kv_write``
    (``full_attention.py:146-149``); quantises for an fp8 pool."""
    if not k.is_cuda:
        raise RuntimeError("write_kv runs only on ROCm devices")
    if k.shape != v.shape or k.dim() != 3 or k.shape[1:] != layer_k_buffer.shape[1:]:
        raise ValueError(f"k/v {tuple(k.shape)} do not match pool rows "
                         f"{tuple(layer_k_buffer.shape[1:])}")
    src = {torch.bfloat16: _native.TF_DTYPE_BF16, torch.float32: _native.TF_DTYPE_FP32}
    if k.dtype not in src or v.dtype != k.dtype:
        raise NotImplementedError(f"k/v dtype {k.dtype}")
    kv_dtype = _KV_DTYPES.get(layer_k_buffer.dtype)
    if kv_dtype is None:
        raise NotImplementedError(f"pool dtype {layer_k_buffer.dtype}")
    if not (layer_k_buffer.is_contiguous() and layer_v_buffer.is_contiguous()):
        raise ValueError("KV pools must be contiguous")
    if not (k.is_contiguous() and v.is_contiguous()):
        k, v = k.contiguous(), v.contiguous()
    loc = out_cache_loc.to(torch.int64).contiguous()
    if loc.numel() != k.shape[0]:
        raise ValueError(f"out_cache_loc has {loc.numel()} slots for {k.shape[0]} tokens")
    if kv_dtype == _native.TF_DTYPE_FP8_E4M3:
        if k_scale is None or v_scale is None:
            raise ValueError("an fp8 KV pool needs k_scale and v_scale")
        k_scale = k_scale.to(device=k.device, dtype=torch.float32).reshape(1).contiguous()
        v_scale = v_scale.to(device=k.device, dtype=torch.float32).reshape(1).contiguous()
    n_kv, head_dim = k.shape[1], k.shape[2]
    _native.call("tf_kv_write", k.data_ptr(), v.data_ptr(), k.stride(0), src[k.dtype],
                 loc.data_ptr(), loc.numel(), layer_k_buffer.data_ptr(),
                 layer_v_buffer.data_ptr(), layer_k_buffer.shape[0], kv_dtype,
                 _ptr(k_scale), _ptr(v_scale), n_kv, head_dim,
                 torch.cuda.current_stream(k.device).cuda_stream)


def qk_norm_rope_kv_write(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                          q_norm_weight: torch.Tensor, k_norm_weight: torch.Tensor,
                          eps: float, positions: torch.Tensor, inv_freq: torch.Tensor,
                          rotary_dim: int, mrope_section, mrope_interleaved: bool,
                          layer_k_buffer: torch.Tensor, layer_v_buffer: torch.Tensor,
                          out_cache_loc: torch.Tensor,
                          k_scale: Optional[torch.Tensor] = None,
                          v_scale: Optional[torch.Tensor] = None,
                          out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """``q_norm``/``k_norm`` + ``rotary_emb`` + the KV write of
    ``full_attention.py:141-149`` in one ``tf_qk_norm_rope_kv_write`` launch.

    ``q`` is ``[T, Hq, D]`` (any token and head stride, e.g. the q half of the
    gated projection), ``k`` / ``v`` ``[T, Hkv, D]`` bf16; ``positions`` is
    ``[T]`` or ``[3, T]`` (M-RoPE). Returns the normalised, rotated q as a new
    contiguous ``[T, Hq, D]`` bf16 tensor (or writes ``out``); K and V land in
    the pool at ``out_cache_loc``.
    """
    if not q.is_cuda:
        raise RuntimeError("qk_norm_rope_kv_write runs only on ROCm devices")
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise NotImplementedError("q/k/v must be bf16")
    if q.dim() != 3 or k.dim() != 3 or k.shape != v.shape or q.shape[0] != k.shape[0]:
        raise ValueError(f"bad q/k/v shapes {tuple(q.shape)} {tuple(k.shape)} {tuple(v.shape)}")
    T, hq, d = q.shape
    hkv = k.shape[1]
    if k.shape[2] != d or layer_k_buffer.shape[1:] != (hkv, d):
        raise ValueError(f"k {tuple(k.shape)} does not match pool rows {tuple(layer_k_buffer.shape[1:])}")
    if q.stride(2) != 1:
        raise ValueError("q rows must be contiguous along head_dim")
    if k.stride(2) != 1 or k.stride(1) != d or v.stride(2) != 1 or v.stride(1) != d:
        k, v = k.contiguous(), v.contiguous()
    kv_dtype = _KV_DTYPES.get(layer_k_buffer.dtype)
    if kv_dtype is None:
        raise NotImplementedError(f"pool dtype {layer_k_buffer.dtype}")
    if not (layer_k_buffer.is_contiguous() and layer_v_buffer.is_contiguous()):
        raise ValueError("KV pools must be contiguous")
    if kv_dtype == _native.TF_DTYPE_FP8_E4M3:
        if k_scale is None or v_scale is None:
            raise ValueError("an fp8 KV pool needs k_scale and v_scale")
        k_scale = k_scale.to(device=q.device, dtype=torch.float32).reshape(1).contiguous()
        v_scale = v_scale.to(device=q.device, dtype=torch.float32).reshape(1).contiguous()
    loc = out_cache_loc.to(device=q.device, dtype=torch.int64).contiguous()
    if loc.numel() != T:
        raise ValueError(f"out_cache_loc has {loc.numel()} slots for {T} tokens")
    pos = positions.to(device=q.device, dtype=torch.int64)
    if pos.dim() == 1:
        pos = pos.reshape(1, -1)
    if pos.dim() != 2 or pos.shape[0] not in (1, 3) or pos.shape[1] != T:
        raise ValueError(f"positions {tuple(positions.shape)} for {T} tokens")
    pos = pos.contiguous()
    qw = q_norm_weight.to(device=q.device, dtype=torch.float32).contiguous()
    kw = k_norm_weight.to(device=q.device, dtype=torch.float32).contiguous()
    freqs = inv_freq.to(device=q.device, dtype=torch.float32).contiguous()
    if freqs.numel() != rotary_dim // 2:
        raise ValueError(f"inv_freq has {freqs.numel()} entries for rotary_dim {rotary_dim}")
    sec = list(mrope_section) if mrope_section is not None else [0, 0, 0]
    if out is None:
        out = torch.empty((T, hq, d), dtype=torch.bfloat16, device=q.device)
    _native.call("tf_qk_norm_rope_kv_write", q.data_ptr(), q.stride(0), q.stride(1),
                 k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0), T, hq, hkv, d,
                 qw.data_ptr(), kw.data_ptr(), float(eps), pos.data_ptr(), pos.shape[0],
                 pos.stride(0), freqs.data_ptr(), rotary_dim, sec[0], sec[1], sec[2],
                 int(bool(mrope_interleaved)), out.data_ptr(), out.stride(0), loc.data_ptr(),
                 layer_k_buffer.data_ptr(), layer_v_buffer.data_ptr(),
                 layer_k_buffer.shape[0], kv_dtype, _ptr(k_scale), _ptr(v_scale),
                 torch.cuda.current_stream(q.device).cuda_stream)
    return out
