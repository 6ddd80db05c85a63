"""Host-side mirror of the reference sampler interface over the HIP engine.

Reference interface (llm-rs, Rust):
  llm-core/src/types.rs:176-196   SampleParams {temperature, top_p, top_k,
                                  repetition_penalty, max_new_tokens}
  llm-core/src/backend.rs:23-24   LlmBackend::sample(logits, params, history)
                                  -> Result<TokenId>
  llm-core/src/sampler.rs:25-125  sample_logits(logits, params, history)
  llm-core/src/sampler.rs:219-228 sample(logits, temperature) -> u32
Here the same names take torch CUDA tensors (device memory) and an explicit
uniform per row instead of rand::thread_rng.  `HipSampler.sample_batch` is the
batched call the scheduler makes once per step instead of scheduler.rs:138-145.
PyTorch only provides device memory and the stream; every computation runs in
libllmk_sampler.so.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Optional, Sequence

import numpy as np
import torch

from . import _lib


class SamplerError(RuntimeError):
    """Raised for a non-zero status of the C ABI (the reference's anyhow::Error)."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"llmk error {code}: {msg}")
        self.code = code


@dataclass
class SampleParams:
    """llm-core/src/types.rs:176-196, plus the engine's extension fields."""

    temperature: float = 1.0
    top_p: float = 1.0
    top_k: int = 0
    repetition_penalty: float = 1.0
    max_new_tokens: int = 512
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0
    min_p: float = 0.0


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


@dataclass
class BatchResult:
    tokens: torch.Tensor
    ids: Optional[torch.Tensor] = None
    probs: Optional[torch.Tensor] = None
    count: Optional[torch.Tensor] = None


@dataclass
class DeviceBatch:
    """Device-resident inputs of one sampling step (all torch CUDA tensors)."""

    logits: torch.Tensor                      # [B, >=V] float32, bfloat16 or float16
    uniforms: torch.Tensor                    # [B] float32
    vocab: Optional[int] = None
    temperature: Optional[torch.Tensor] = None
    top_k: Optional[torch.Tensor] = None      # int32
    top_p: Optional[torch.Tensor] = None
    min_p: Optional[torch.Tensor] = None
    repetition_penalty: Optional[torch.Tensor] = None
    presence_penalty: Optional[torch.Tensor] = None
    frequency_penalty: Optional[torch.Tensor] = None
    hist_offsets: Optional[torch.Tensor] = None  # int32/uint32 [B+1]
    hist_tokens: Optional[torch.Tensor] = None   # int32/uint32
    allow_mask: Optional[torch.Tensor] = None    # int32/uint32 [B, words]
    hist_lengths: Optional[torch.Tensor] = None  # int32/uint32 [B]: per-row buffers
    softcap: float = 0.0  # > 0: the logits are the lm_head output before final_logit_softcapping
    hist_counts: Optional[torch.Tensor] = None  # int32/uint32, like hist_tokens: occurrences


def _on_device(dev: torch.device, **tensors) -> None:
    """Every tensor handed to the C ABI must live on the logits' GPU: a host
    pointer or another device's pointer would reach a kernel."""
    if dev.type != "cuda":
        raise SamplerError(_lib.LLMK_ERR_INVALID_ARGUMENT, "logits must be a CUDA (HIP) tensor")
    for name, t in tensors.items():
        if t is not None and t.device != dev:
            raise SamplerError(_lib.LLMK_ERR_INVALID_ARGUMENT,
                               f"{name} is on {t.device}, the logits on {dev}")


def _rows(t: torch.Tensor) -> bool:
    """A [rows, columns] tensor with unit stride along the columns.  torch
    gives a dimension of size 1 any stride (a one-row view of a 1-D tensor
    has stride 0 across rows), so such a dimension is not checked."""
    return t.dim() == 2 and (t.stride(1) == 1 or t.shape[1] <= 1)


def _row_stride(t: torch.Tensor) -> int:
    """Elements from one row's start to the next; a single row is read as
    packed whatever stride torch gives its size-1 dimension."""
    return t.stride(0) if t.shape[0] > 1 else max(t.stride(0), t.shape[1])


def _flat(name: str, t: Optional[torch.Tensor], dtypes) -> None:
    """Per-row arrays are read as dense vectors of one element type."""
    if t is not None and (t.dtype not in dtypes or not t.is_contiguous()):
        raise SamplerError(_lib.LLMK_ERR_INVALID_ARGUMENT,
                           f"{name} must be a contiguous {' or '.join(map(str, dtypes))} tensor")


_I32 = (torch.int32,)
_F32 = (torch.float32,)


def _batch_args(db: DeviceBatch, out_tokens: torch.Tensor,
                out_ids: Optional[torch.Tensor], out_probs: Optional[torch.Tensor],
                out_count: Optional[torch.Tensor]) -> "_lib.SampleBatchArgs":
    """llmk_sample_batch_args for db, after checking every tensor's device,
    element type and layout (nothing is converted, so nothing temporary has
    to outlive the call)."""
    lg = db.logits
    if lg.dtype == torch.float32:
        dt = _lib.LLMK_F32
    elif lg.dtype == torch.bfloat16:
        dt = _lib.LLMK_BF16
    elif lg.dtype == torch.float16:
        dt = _lib.LLMK_F16
    else:
        raise SamplerError(_lib.LLMK_ERR_INVALID_ARGUMENT,
                           "logits must be float32, bfloat16 or float16")
    if not _rows(lg):
        raise SamplerError(_lib.LLMK_ERR_INVALID_ARGUMENT,
                           "logits must be [batch, >= vocab] with unit stride along the vocabulary")
    fields = dict(uniforms=db.uniforms, temperature=db.temperature, top_k=db.top_k,
                  top_p=db.top_p, min_p=db.min_p, repetition_penalty=db.repetition_penalty,
                  presence_penalty=db.presence_penalty, frequency_penalty=db.frequency_penalty,
                  hist_offsets=db.hist_offsets, hist_tokens=db.hist_tokens,
                  allow_mask=db.allow_mask, hist_lengths=db.hist_lengths,
                  hist_counts=db.hist_counts, out_tokens=out_tokens, out_ids=out_ids, out_probs=out_probs,
                  out_count=out_count)
    _on_device(lg.device, **fields)
    if db.uniforms is None:
        raise SamplerError(_lib.LLMK_ERR_INVALID_ARGUMENT, "uniforms are required")
    for name in ("uniforms", "temperature", "top_p", "min_p", "repetition_penalty",
                 "presence_penalty", "frequency_penalty", "out_probs"):
        _flat(name, fields[name], _F32)
    for name in ("top_k", "out_tokens", "out_ids", "out_count"):
        _flat(name, fields[name], _I32)
    for name in ("hist_offsets", "hist_tokens", "allow_mask", "hist_lengths", "hist_counts"):
        _flat(name, fields[name], _I32 + (getattr(torch, "uint32", torch.int32),))
    B = lg.shape[0]
    V = db.vocab if db.vocab is not None else lg.shape[1]
    a = _lib.SampleBatchArgs()
    a.logits = lg.data_ptr()
    a.dtype = dt
    a.batch = B
    a.vocab = V
    a.row_stride = _row_stride(lg)
    a.temperature = _ptr(db.temperature)
    a.top_k = _ptr(db.top_k)
    a.top_p = _ptr(db.top_p)
    a.min_p = _ptr(db.min_p)
    a.repetition_penalty = _ptr(db.repetition_penalty)
    a.presence_penalty = _ptr(db.presence_penalty)
    a.frequency_penalty = _ptr(db.frequency_penalty)
    a.hist_offsets = _ptr(db.hist_offsets)
    a.hist_tokens = _ptr(db.hist_tokens)
    a.allow_mask = _ptr(db.allow_mask)
    a.mask_words_per_row = 0 if db.allow_mask is None else db.allow_mask.shape[1]
    a.uniforms = _ptr(db.uniforms)
    a.out_tokens = _ptr(out_tokens)
    a.out_ids = _ptr(out_ids)
    a.out_probs = _ptr(out_probs)
    cap = 0
    if out_ids is not None:
        cap = out_ids.shape[1]
    elif out_probs is not None:
        cap = out_probs.shape[1]
    a.out_cap = cap
    a.out_count = _ptr(out_count)
    a.hist_lengths = _ptr(db.hist_lengths)
    a.softcap = float(db.softcap or 0.0)
    a.hist_counts = _ptr(db.hist_counts)
    return a


def sample_batch_static(db: DeviceBatch, out_tokens: torch.Tensor,
                        out_ids: Optional[torch.Tensor] = None,
                        out_probs: Optional[torch.Tensor] = None,
                        out_count: Optional[torch.Tensor] = None,
                        status: Optional[torch.Tensor] = None,
                        stream: Optional[torch.cuda.Stream] = None) -> None:
    """llmk_sample_batch_static: the batched call without a handle and without
    allocating (batch <= 256, vocab <= 262144), on the logits' device.
    `status`: optional int32 [1] device tensor the call ORs its status bits
    into.  Calls that overlap on one GPU race on its static workspace."""
    lib = _lib.load()
    a = _batch_args(db, out_tokens, out_ids, out_probs, out_count)
    _on_device(db.logits.device, status=status)
    _flat("status", status, _I32)
    st = stream if stream is not None else torch.cuda.current_stream(db.logits.device)
    with torch.cuda.device(db.logits.device):
        rc = lib.llmk_sample_batch_static(ctypes.byref(a), _ptr(status),
                                          ctypes.c_void_p(st.cuda_stream))
    if rc != 0:
        raise SamplerError(rc, _lib.last_error())


class HipSampler:
    """Owns an llmk_sampler handle (device workspace) on one GPU."""

    def __init__(self, max_batch: int, max_vocab: int, device: int = 0):
        self._lib = _lib.load()
        self.device = device
        self.max_batch = max_batch
        self.max_vocab = max_vocab
        h = ctypes.c_void_p()
        rc = self._lib.llmk_sampler_create(ctypes.byref(h), device, max_batch, max_vocab)
        if rc != 0:
            raise SamplerError(rc, _lib.last_error())
        self._h = h

    def close(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            self._lib.llmk_sampler_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- the batched call -------------------------------------------------
    def launch(self, db: DeviceBatch, out_tokens: torch.Tensor,
               out_ids: Optional[torch.Tensor] = None,
               out_probs: Optional[torch.Tensor] = None,
               out_count: Optional[torch.Tensor] = None,
               stream: Optional[torch.cuda.Stream] = None) -> None:
        """Enqueue one batched sampling call; no allocation, no sync."""
        a = _batch_args(db, out_tokens, out_ids, out_probs, out_count)
        self.launch_prepared(a, self._stream(db.logits, stream))

    def prepare(self, db: DeviceBatch, out_tokens: torch.Tensor,
                out_ids: Optional[torch.Tensor] = None,
                out_probs: Optional[torch.Tensor] = None,
                out_count: Optional[torch.Tensor] = None) -> "_lib.SampleBatchArgs":
        """The checked llmk_sample_batch_args of a call, for a caller that
        launches the same buffers many times (launch_prepared)."""
        return _batch_args(db, out_tokens, out_ids, out_probs, out_count)

    def launch_prepared(self, a: "_lib.SampleBatchArgs", stream: torch.cuda.Stream) -> None:
        """llmk_sample_batch on arguments from prepare(); the tensors they
        point at must still be alive."""
        rc = self._lib.llmk_sample_batch(self._h, ctypes.byref(a),
                                         ctypes.c_void_p(stream.cuda_stream))
        if rc != 0:
            raise SamplerError(rc, _lib.last_error())

    def sample_batch(self, db: DeviceBatch, out_cap: int = 0) -> BatchResult:
        B = db.logits.shape[0]
        dev = db.logits.device
        tok = torch.empty(B, dtype=torch.int32, device=dev)
        ids = probs = None
        if out_cap:
            ids = torch.empty(B, out_cap, dtype=torch.int32, device=dev)
            probs = torch.empty(B, out_cap, dtype=torch.float32, device=dev)
        cnt = torch.empty(B, dtype=torch.int32, device=dev)
        self.launch(db, tok, ids, probs, cnt)
        return BatchResult(tok, ids, probs, cnt)

    def status(self) -> int:
        v = ctypes.c_uint32()
        st = torch.cuda.current_stream(self.device)
        rc = self._lib.llmk_sampler_status(self._h, ctypes.c_void_p(st.cuda_stream), ctypes.byref(v))
        if rc != 0:
            raise SamplerError(rc, _lib.last_error())
        return v.value

    # ---- mask forms (sampler.rs:160-216), batched, in place --------------
    def _stream(self, logits: torch.Tensor, stream: Optional[torch.cuda.Stream]):
        return stream if stream is not None else torch.cuda.current_stream(logits.device)

    @staticmethod
    def _keep(st, *tmps: torch.Tensor) -> None:
        """Converted copies are freed when the wrapper returns, while the
        kernel may still be queued on `st`: tell the caching allocator."""
        for t in tmps:
            t.record_stream(st)

    def _mask(self, fn: str, logits: torch.Tensor, param: torch.Tensor, dtype: torch.dtype,
              stream: Optional[torch.cuda.Stream]) -> None:
        if logits.dtype != torch.float32 or not _rows(logits):
            raise SamplerError(_lib.LLMK_ERR_INVALID_ARGUMENT,
                               "logits must be a row-major float32 [batch, vocab] tensor")
        _on_device(logits.device, param=param)
        if param.numel() != logits.shape[0]:
            raise SamplerError(_lib.LLMK_ERR_INVALID_ARGUMENT, "one parameter per row")
        st = self._stream(logits, stream)
        p = param.to(dtype).contiguous()
        rc = getattr(self._lib, fn)(self._h, logits.data_ptr(), logits.shape[0], logits.shape[1],
                                    _row_stride(logits), p.data_ptr(),
                                    ctypes.c_void_p(st.cuda_stream))
        if rc != 0:
            raise SamplerError(rc, _lib.last_error())
        self._keep(st, p)

    def apply_top_k(self, logits: torch.Tensor, top_k: torch.Tensor,
                    stream: Optional[torch.cuda.Stream] = None) -> None:
        """sampler.rs:160-173 on every row: logits [B, V] float32, top_k [B] int32."""
        self._mask("llmk_apply_top_k", logits, top_k, torch.int32, stream)

    def apply_top_p(self, logits: torch.Tensor, top_p: torch.Tensor,
                    stream: Optional[torch.cuda.Stream] = None) -> None:
        """sampler.rs:176-216 on every row: logits [B, V] float32, top_p [B] float32."""
        self._mask("llmk_apply_top_p", logits, top_p, torch.float32, stream)

    def apply_logit_bias(self, logits: torch.Tensor, offsets: torch.Tensor,
                         tokens: torch.Tensor, values: torch.Tensor,
                         stream: Optional[torch.cuda.Stream] = None) -> None:
        """logits[b, tokens[j]] += values[j] for j in offsets[b]..offsets[b+1]
        (the formula of mlc_parity.rs:1060-1072), in place on [B, V] float32."""
        if logits.dtype != torch.float32 or not _rows(logits):
            raise SamplerError(_lib.LLMK_ERR_INVALID_ARGUMENT,
                               "logits must be a row-major float32 [batch, vocab] tensor")
        _on_device(logits.device, offsets=offsets, tokens=tokens, values=values)
        if offsets.numel() != logits.shape[0] + 1 or tokens.numel() != values.numel():
            raise SamplerError(_lib.LLMK_ERR_INVALID_ARGUMENT,
                               "offsets must hold batch + 1 entries, tokens and values one per pair")
        off = offsets.to(torch.int32).contiguous()
        tok = tokens.to(torch.int32).contiguous()
        val = values.to(torch.float32).contiguous()
        st = self._stream(logits, stream)
        rc = self._lib.llmk_apply_logit_bias(self._h, logits.data_ptr(), logits.shape[0],
                                             logits.shape[1], _row_stride(logits), off.data_ptr(),
                                             tok.data_ptr(), val.data_ptr(),
                                             ctypes.c_void_p(st.cuda_stream))
        if rc != 0:
            raise SamplerError(rc, _lib.last_error())
        self._keep(st, off, tok, val)

    def history_append(self, hist_offsets: torch.Tensor, hist_lengths: torch.Tensor,
                       hist_tokens: torch.Tensor, capacity: int, tokens: torch.Tensor,
                       stream: Optional[torch.cuda.Stream] = None) -> None:
        """scheduler.rs:147 on the device: append tokens[b] to row b's history
        buffer (int32 tensors, updated in place)."""
        for t in (hist_offsets, hist_lengths, hist_tokens, tokens):
            if t.dtype != torch.int32 or not t.is_contiguous():
                raise SamplerError(_lib.LLMK_ERR_INVALID_ARGUMENT,
                                   "history arrays and tokens must be contiguous int32")
        _on_device(tokens.device, hist_offsets=hist_offsets, hist_lengths=hist_lengths,
                   hist_tokens=hist_tokens)
        B = tokens.shape[0]
        if hist_offsets.numel() < B or hist_lengths.numel() < B:
            raise SamplerError(_lib.LLMK_ERR_INVALID_ARGUMENT,
                               "hist_offsets and hist_lengths need one entry per row")
        st = self._stream(tokens, stream)
        rc = self._lib.llmk_history_append(self._h, tokens.shape[0], hist_offsets.data_ptr(),
                                           hist_lengths.data_ptr(), hist_tokens.data_ptr(),
                                           capacity, tokens.data_ptr(),
                                           ctypes.c_void_p(st.cuda_stream))
        if rc != 0:
            raise SamplerError(rc, _lib.last_error())

    def history_count_append(self, hist_offsets: torch.Tensor, hist_lengths: torch.Tensor,
                             hist_tokens: torch.Tensor, hist_counts: torch.Tensor,
                             capacity: int, tokens: torch.Tensor,
                             stream: Optional[torch.cuda.Stream] = None) -> None:
        """scheduler.rs:147 on a count-table history: token b joins row b's
        sorted distinct tokens (count 1) or raises its count (int32 tensors,
        updated in place)."""
        for t in (hist_offsets, hist_lengths, hist_tokens, hist_counts, tokens):
            if t.dtype != torch.int32 or not t.is_contiguous():
                raise SamplerError(_lib.LLMK_ERR_INVALID_ARGUMENT,
                                   "history arrays, counts and tokens must be contiguous int32")
        _on_device(tokens.device, hist_offsets=hist_offsets, hist_lengths=hist_lengths,
                   hist_tokens=hist_tokens, hist_counts=hist_counts)
        B = tokens.shape[0]
        if hist_offsets.numel() < B or hist_lengths.numel() < B:
            raise SamplerError(_lib.LLMK_ERR_INVALID_ARGUMENT,
                               "hist_offsets and hist_lengths need one entry per row")
        if hist_counts.numel() < hist_tokens.numel():
            raise SamplerError(_lib.LLMK_ERR_INVALID_ARGUMENT,
                               "hist_counts needs an entry per hist_tokens entry")
        st = self._stream(tokens, stream)
        rc = self._lib.llmk_history_count_append(
            self._h, B, hist_offsets.data_ptr(), hist_lengths.data_ptr(),
            hist_tokens.data_ptr(), hist_counts.data_ptr(), capacity, tokens.data_ptr(),
            ctypes.c_void_p(st.cuda_stream))
        if rc != 0:
            raise SamplerError(rc, _lib.last_error())

    # ---- speculative-decoding verification (docs/mlc-contracts.md:83-84) --
    def verify_batch(self, ids: torch.Tensor, probs: torch.Tensor, counts: torch.Tensor,
                     draft_tokens: torch.Tensor, draft_probs: torch.Tensor,
                     u_accept: torch.Tensor, u_resample: torch.Tensor,
                     vocab: Optional[int] = None,
                     stream: Optional[torch.cuda.Stream] = None):
        """llmk_verify_batch: row b accepts draft_tokens[b] against the target
        distribution given by the kept list ids/probs[b, :counts[b]] (what
        sample_batch returns with out_cap = ids.shape[1]), or resamples from
        max(p - q, 0) with q = draft_probs[b].  Returns (tokens, accepted)."""
        B, cap = ids.shape
        V = vocab if vocab is not None else draft_probs.shape[1]
        _on_device(ids.device, probs=probs, counts=counts, draft_tokens=draft_tokens,
                   draft_probs=draft_probs, u_accept=u_accept, u_resample=u_resample)
        for name, t, dts in (("ids", ids, _I32), ("probs", probs, _F32), ("counts", counts, _I32),
                             ("draft_tokens", draft_tokens, _I32), ("u_accept", u_accept, _F32),
                             ("u_resample", u_resample, _F32)):
            _flat(name, t, dts)
        if draft_probs.dtype != torch.float32 or not _rows(draft_probs):
            raise SamplerError(_lib.LLMK_ERR_INVALID_ARGUMENT,
                               "draft_probs must be a row-major float32 [batch, >= vocab] tensor")
        if probs.shape != ids.shape or draft_probs.shape[0] != B or counts.numel() != B:
            raise SamplerError(_lib.LLMK_ERR_INVALID_ARGUMENT, "inconsistent shapes")
        if V > draft_probs.shape[1]:
            # the kernel reads q[id] for every id < vocab of the last row too
            raise SamplerError(_lib.LLMK_ERR_INVALID_ARGUMENT,
                               f"vocab {V} above draft_probs' {draft_probs.shape[1]} columns")
        tok = torch.empty(B, dtype=torch.int32, device=ids.device)
        acc = torch.empty(B, dtype=torch.int32, device=ids.device)
        st = self._stream(ids, stream)
        rc = self._lib.llmk_verify_batch(self._h, B, V, ids.data_ptr(), probs.data_ptr(), cap,
                                         counts.data_ptr(), draft_tokens.data_ptr(),
                                         draft_probs.data_ptr(), _row_stride(draft_probs),
                                         u_accept.data_ptr(), u_resample.data_ptr(),
                                         tok.data_ptr(), acc.data_ptr(),
                                         ctypes.c_void_p(st.cuda_stream))
        if rc != 0:
            raise SamplerError(rc, _lib.last_error())
        return tok, acc

    # ---- the per-row reference call (LlmBackend::sample) ------------------
    def sample(self, logits: torch.Tensor, params: SampleParams,
               token_history: Sequence[int], u: float) -> int:
        """sampler.rs:25-125 for one row; raises SamplerError on empty logits."""
        if logits.numel() == 0:
            raise SamplerError(_lib.LLMK_ERR_EMPTY_LOGITS, "Empty logits passed to sampler")
        db = device_batch_from_params(logits.reshape(1, -1), [params], [list(token_history)], [u])
        return int(self.sample_batch(db).tokens[0].item())


def device_batch_from_params(logits: torch.Tensor, params: Sequence[SampleParams],
                             histories: Sequence[Sequence[int]], uniforms: Sequence[float],
                             allow_mask: Optional[np.ndarray] = None) -> DeviceBatch:
    """Pack per-row SampleParams / histories into device arrays."""
    dev = logits.device
    f = lambda xs: torch.tensor(np.asarray(xs, dtype=np.float32), device=dev)
    offs = np.zeros(len(histories) + 1, dtype=np.int64)
    for i, h in enumerate(histories):
        offs[i + 1] = offs[i] + len(h)
    toks = np.concatenate([np.asarray(h, dtype=np.uint32) for h in histories]) if offs[-1] else np.zeros(1, np.uint32)
    return DeviceBatch(
        logits=logits,
        uniforms=f(uniforms),
        temperature=f([p.temperature for p in params]),
        top_k=torch.tensor(np.asarray([p.top_k for p in params], dtype=np.int32), device=dev),
        top_p=f([p.top_p for p in params]),
        min_p=f([p.min_p for p in params]),
        repetition_penalty=f([p.repetition_penalty for p in params]),
        presence_penalty=f([p.presence_penalty for p in params]),
        frequency_penalty=f([p.frequency_penalty for p in params]),
        hist_offsets=torch.tensor(offs.astype(np.int32), device=dev),
        hist_tokens=torch.tensor(toks.view(np.int32), device=dev),
        allow_mask=None if allow_mask is None else torch.tensor(allow_mask.view(np.int32), device=dev),
    )


def sample_logits(sampler: HipSampler, logits: torch.Tensor, params: SampleParams,
                  token_history: Sequence[int], u: float) -> int:
    """Free-function form of sampler.rs:25 sample_logits."""
    return sampler.sample(logits, params, token_history, u)


def sample(sampler: HipSampler, logits: torch.Tensor, temperature: float, u: float) -> int:
    """sampler.rs:219-228: temperature only, unwrap_or(0) on error."""
    try:
        return sampler.sample(logits, SampleParams(temperature=temperature), [], u)
    except SamplerError:
        return 0


def apply_top_k(sampler: HipSampler, logits: torch.Tensor, top_k: int) -> None:
    """Free-function form of sampler.rs:160 apply_top_k for one row, in place."""
    lg = logits.view(1, -1)
    sampler.apply_top_k(lg, torch.tensor([min(int(top_k), 2**31 - 1)], dtype=torch.int32,
                                         device=logits.device))


def apply_top_p(sampler: HipSampler, logits: torch.Tensor, top_p: float) -> None:
    """Free-function form of sampler.rs:176 apply_top_p for one row, in place."""
    lg = logits.view(1, -1)
    sampler.apply_top_p(lg, torch.tensor([top_p], dtype=torch.float32, device=logits.device))
