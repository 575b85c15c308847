"""RustQwenDecoder on MI355X: the reference's native decoder API over libtbhip.so.

Mirrors the reference's RustQwenDecoder pyclass (src/llm/decoder.rs:176-1020)
and its factory create_rust_qwen_decoder (python/torchburn/quantization.py:575-647):
same constructor arguments, layer tensor order and method names.  Tensors may be
torch (CPU or GPU) or numpy arrays; they are copied to the GPU once at
construction, as the reference copies them into Rust-owned memory.
"""
from __future__ import annotations

import ctypes as C
from typing import Any, List, Optional, Sequence, Tuple

import numpy as np

from . import _lib

RECENT_WINDOW = 64   # repetition-penalty window (src/llm/decoder.rs:837-850)


class _Config(C.Structure):
    _fields_ = [("num_layers", C.c_int64), ("hidden_size", C.c_int64),
                ("intermediate_size", C.c_int64), ("num_heads", C.c_int64),
                ("num_kv_heads", C.c_int64), ("head_dim", C.c_int64),
                ("vocab_size", C.c_int64), ("group_size", C.c_int64),
                ("max_seq_len", C.c_int64), ("rms_norm_eps", C.c_double),
                ("rope_theta", C.c_double), ("weight_bits", C.c_int32),
                ("lm_head_bits", C.c_int32)]


def _bind():
    L = _lib.lib()
    if getattr(L, "_tb_decoder_bound", False):
        return L
    p, i64 = C.c_void_p, C.c_int64
    sigs = {
        "tb_decoder_create": [C.POINTER(_Config), p, p, p, p, C.POINTER(p)],
        "tb_decoder_set_layer": [p, i64] + [p] * 13,
        "tb_decoder_step": [p, i64, i64, p, C.POINTER(i64)],
        "tb_decoder_decode_and_sample": [p, i64, i64, C.c_float, i64, C.c_float, p, i64,
                                         C.c_float, C.POINTER(i64)],
        "tb_decoder_generate": [p, i64, i64, i64, i64, p, C.POINTER(i64), C.POINTER(i64)],
        "tb_decoder_generate_sampled": [p, i64, i64, i64, C.c_float, i64, C.c_float, C.c_float,
                                        i64, p, i64, p, C.POINTER(i64), C.POINTER(i64)],
        "tb_decoder_prefill": [p, p, i64, i64, C.POINTER(i64)],
        "tb_decoder_verify": [p, i64, p, i64, p],
        "tb_decoder_speculative_accept": [p, i64, p, i64, p, C.c_float, C.c_float,
                                          C.POINTER(i64), C.POINTER(i64)],
        "tb_speculative_accept_rows": [p, p, p, i64, i64, C.c_float, C.c_float, p, i64,
                                       C.POINTER(i64), C.POINTER(i64)],
        "tb_decoder_reset_kv": [p],
        "tb_decoder_copy_kv": [p, i64, p, p, i64, i64],
        "tb_decoder_kv_len": [p, C.POINTER(i64)],
        "tb_decoder_get_logits": [p, p],
        "tb_decoder_set_seed": [p, C.c_uint64],
        "tb_decoder_set_rope_tables": [p, p, p, i64, i64],
        "tb_decoder_set_attention_cap": [p, i64],
        "tb_decoder_time_greedy": [p, i64, i64, i64, C.POINTER(C.c_float)],
        "tb_decoder_destroy": [p],
    }
    for name, args in sigs.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = C.c_int
    L.tb_spec_uniform.restype = C.c_double
    L.tb_spec_uniform.argtypes = [C.c_uint64, C.c_uint64]
    L._tb_decoder_bound = True
    return L


def speculative_accept_rows(target_rows, draft_tokens, draft_probs, u, temperature: float = 1.0,
                            top_p: float = 1.0) -> Tuple[int, int]:
    """The acceptance of speculative_accept over given target logits rows [K, V]
    with the uniforms u (decoder.rs:608-726)."""
    rows = np.ascontiguousarray(np.asarray(target_rows, dtype=np.float32))
    k, v = (rows.shape if rows.ndim == 2 else (0, rows.size))
    arr = np.asarray(list(draft_tokens), dtype=np.int64)
    probs = np.ascontiguousarray(np.asarray(draft_probs, dtype=np.float32).reshape(-1))
    uu = np.ascontiguousarray(np.asarray(list(u), dtype=np.float64))
    a, b = C.c_int64(), C.c_int64()
    _lib.check(_bind().tb_speculative_accept_rows(
        rows.ctypes.data, arr.ctypes.data, probs.ctypes.data, k, v, float(temperature),
        float(top_p), uu.ctypes.data if uu.size else None, uu.size, C.byref(a), C.byref(b)))
    return int(a.value), int(b.value)


def spec_uniform(seed: int, counter: int) -> float:
    """The decoder's f64 uniform of draw ``counter`` under ``seed``."""
    return float(_bind().tb_spec_uniform(int(seed) & (2 ** 64 - 1), int(counter) & (2 ** 64 - 1)))


def decoder_symbols() -> list:
    return ["tb_decoder_create", "tb_decoder_set_layer", "tb_decoder_step",
            "tb_decoder_decode_and_sample", "tb_decoder_generate", "tb_decoder_prefill",
            "tb_decoder_reset_kv", "tb_decoder_copy_kv", "tb_decoder_kv_len",
            "tb_decoder_get_logits", "tb_decoder_set_seed", "tb_decoder_time_greedy",
            "tb_decoder_destroy", "tb_decoder_generate_sampled", "tb_decoder_verify",
            "tb_decoder_speculative_accept", "tb_speculative_accept_rows", "tb_spec_uniform",
            "tb_decoder_set_rope_tables", "tb_decoder_set_attention_cap"]


_NP_TO_TORCH = {"float32": "float32", "uint8": "uint8", "int8": "int8", "int64": "int64"}


def _as_buffer(t: Any, dtype=None, numel: Optional[int] = None, what: str = "tensor"):
    """(pointer, keep-alive object, dtype name) of a contiguous tensor/array.

    ``dtype`` (a numpy dtype) converts the data first, for torch tensors as for
    arrays; ``numel`` is the element count the C side will read, checked here
    because the C ABI receives no lengths (a short or mis-typed buffer would be
    over-read), as the reference's typed_slice rejects a wrong element size
    (src/llm/decoder.rs:77-89)."""
    if t is None:
        return None, None, None
    try:
        import torch
        if isinstance(t, torch.Tensor):
            t = t.detach()
            if dtype is not None:
                t = t.to(getattr(torch, _NP_TO_TORCH[np.dtype(dtype).name]))
            t = t.contiguous()
            name = str(t.dtype).replace("torch.", "")
            if numel is not None and t.numel() != numel:
                raise _lib.UnsupportedOpError(
                    f"{_lib.UNSUPPORTED_MARKER} {what}: expected {numel} elements, got {t.numel()}")
            return t.data_ptr(), t, name
    except ImportError:
        pass
    a = np.ascontiguousarray(t if dtype is None else np.asarray(t, dtype=dtype))
    if numel is not None and a.size != numel:
        raise _lib.UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} {what}: expected {numel} elements, got {a.size}")
    return a.ctypes.data, a, str(a.dtype)


def _bits_of(dtype: str) -> int:
    bits = {"uint8": 4, "int8": 8, "float32": 32}.get(dtype)
    if bits is None:
        raise _lib.UnsupportedOpError(
            f"{_lib.UNSUPPORTED_MARKER} projection weights must be uint8 (INT4 packed), int8 or "
            f"float32, got {dtype}")
    return bits


def _proj_sizes(bits: int, n: int, k: int, gs: int) -> Tuple[int, int]:
    """(weight elements, scale elements) the decoder reads for a projection [n, k]."""
    if bits == 4:
        return n * ((k + 1) // 2), n * (k // gs)
    if bits == 8:
        return n * k, n
    return n * k, 0


def _row_scales(s: Any, n: int):
    """INT8 scales as n per-row values: a 1-element (per-tensor) scale is repeated."""
    a = s.detach().float().reshape(-1).cpu().numpy() if hasattr(s, "detach") else \
        np.asarray(s, np.float32).reshape(-1)
    return np.repeat(a, n) if a.size == 1 and n != 1 else a


def rotary_tables_f32(max_seq: int, head_dim: int, theta: float) -> Tuple[np.ndarray, np.ndarray]:
    """cos / sin [max_seq, head_dim] exactly as the reference's per-layer Python
    path builds them (RotaryEmbedding, python/torchburn/llm/model.py:108-122):
    inv_freq = 1 / theta ** (arange(0, d, 2) / d) in float32, the angle
    t * inv_freq as a float32 product, cos / sin in float32, halves duplicated.
    The native decoder instead builds its tables in f64 (decoder.rs:334-350);
    the two differ by up to ~1e-4 at positions in the thousands."""
    import torch
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    t = torch.arange(0, max_seq, dtype=torch.float32)
    freqs = torch.outer(t, inv_freq)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().numpy().astype(np.float32), emb.sin().numpy().astype(np.float32)


class RustQwenDecoder:
    """Device-resident INT4 (or INT8) decoder with the reference's API.

    Constructor arguments are those of RustQwenDecoder::new (decoder.rs:176-212);
    each entry of ``layers_data`` is the reference's 12 (+1 bias) tensors:
    [in_norm, qkv_w, qkv_s, o_w, o_s, post_norm, gate_w, gate_s, up_w, up_s,
    down_w, down_s, (qkv_b)].  Projection format follows the weight dtype
    (uint8 packed nibbles = INT4 grouped, int8 = INT8 per-channel); the lm_head
    may be INT4, INT8 or float32 (``lm_head_s`` None).
    """

    def __init__(self, embed_tokens, layers_data: Sequence[Sequence[Any]], final_norm_w,
                 lm_head_w, lm_head_s, num_layers: int, hidden_size: int,
                 intermediate_size: int, num_heads: int, num_kv_heads: int, head_dim: int,
                 group_size: int = 64, rms_norm_eps: float = 1e-6, max_seq_len: int = 2048,
                 rope_theta: float = 1e6):
        L = _bind()
        self._h = None
        vocab = int(embed_tokens.shape[0])
        H, I, gs = int(hidden_size), int(intermediate_size), int(group_size)
        qd, tq = num_heads * head_dim, (num_heads + 2 * num_kv_heads) * head_dim
        if len(layers_data) != num_layers:
            raise ValueError(f"expected {num_layers} layers, got {len(layers_data)}")
        emb_p, emb_k, _ = _as_buffer(embed_tokens, np.float32, vocab * H, "embed_tokens")
        fn_p, fn_k, _ = _as_buffer(final_norm_w, np.float32, H, "final_norm_w")
        lm_dt = _as_buffer(lm_head_w)[2]
        lmbits = _bits_of(lm_dt)
        lw_n, ls_n = _proj_sizes(lmbits, vocab, H, gs)
        lm_p, lm_k, _ = _as_buffer(lm_head_w, None, lw_n, "lm_head_w")
        if lmbits == 8 and lm_head_s is not None:
            lm_head_s = _row_scales(lm_head_s, vocab)
        ls_p, ls_k, _ = (_as_buffer(lm_head_s, np.float32, ls_n, "lm_head_s")
                         if lm_head_s is not None and lmbits != 32 else (None, None, None))
        wdt = _as_buffer(layers_data[0][1])[2] if num_layers else "uint8"
        wbits = _bits_of(wdt)
        if wbits == 32:
            raise _lib.UnsupportedOpError(
                f"{_lib.UNSUPPORTED_MARKER} decoder projections must be INT4 or INT8")
        cfg = _Config(num_layers, hidden_size, intermediate_size, num_heads, num_kv_heads,
                      head_dim, vocab, group_size, max_seq_len, float(rms_norm_eps),
                      float(rope_theta), wbits, lmbits)
        h = C.c_void_p()
        _lib.check(L.tb_decoder_create(C.byref(cfg), emb_p, fn_p, lm_p, ls_p, C.byref(h)))
        self._h = h
        self.vocab_size = vocab
        self.hidden_size = hidden_size
        self.head_dim = head_dim
        self.num_kv_heads = num_kv_heads
        self.num_layers = num_layers
        self.max_seq_len = max_seq_len
        self.weight_bits = cfg.weight_bits
        self.lm_head_bits = cfg.lm_head_bits
        del emb_k, fn_k, lm_k, ls_k
        # (name, projection rows, K) of the weight / scale pairs in capsule order
        shapes = {1: ("qkv", tq, H), 3: ("o", H, qd), 6: ("gate", I, H), 8: ("up", I, H),
                  10: ("down", H, I)}
        wdtype = np.uint8 if wbits == 4 else np.int8
        for li, caps in enumerate(layers_data):
            if len(caps) < 12:
                raise _lib.UnsupportedOpError(
                    f"{_lib.UNSUPPORTED_MARKER} Each layer requires 12 capsules: input_norm, "
                    "qkv_w, qkv_s, o_w, o_s, post_norm, gate_w, gate_s, up_w, up_s, down_w, down_s")
            bufs = [None] * 12
            for i in (0, 5):
                bufs[i] = _as_buffer(caps[i], np.float32, H, f"layer {li} norm")
            for i, (name, n, k) in shapes.items():
                wn, sn = _proj_sizes(wbits, n, k, gs)
                if _as_buffer(caps[i])[2] != np.dtype(wdtype).name:
                    raise _lib.UnsupportedOpError(
                        f"{_lib.UNSUPPORTED_MARKER} layer {li} {name}_w must be "
                        f"{np.dtype(wdtype).name} like the other projections")
                bufs[i] = _as_buffer(caps[i], None, wn, f"layer {li} {name}_w")
                sc = _row_scales(caps[i + 1], n) if wbits == 8 else caps[i + 1]
                bufs[i + 1] = _as_buffer(sc, np.float32, sn, f"layer {li} {name}_s")
            qkv_b = _as_buffer(caps[12], np.float32, tq, f"layer {li} qkv_b") \
                if len(caps) >= 13 and caps[12] is not None else (None, None, None)
            _lib.check(L.tb_decoder_set_layer(self._h, li, *[b[0] for b in bufs], qkv_b[0]))

    def set_rope_tables(self, cos, sin) -> None:
        """Replace the decoder's f64-built RoPE tables (decoder.rs:334-350) with
        caller-built cos / sin [max_seq_len, head_dim], e.g. rotary_tables_f32(),
        the tables of the reference's per-layer Python path (no reference
        counterpart on RustQwenDecoder)."""
        n = self.max_seq_len * self.head_dim
        cp, ck, _ = _as_buffer(cos, np.float32, n, "cos")
        sp, sk, _ = _as_buffer(sin, np.float32, n, "sin")
        _lib.check(_bind().tb_decoder_set_rope_tables(self._h, cp, sp, self.max_seq_len,
                                                      self.head_dim))
        del ck, sk

    def set_attention_cap(self, cap: int) -> None:
        """Positions a step attends: 0 .. min(p + 1, cap) - 1 at position p.
        The default, 32768, is RustQwenDecoder's native step (decoder.rs:1179-
        1184); 0 scores every position, as the reference's per-layer Python
        path does (no reference counterpart on RustQwenDecoder)."""
        _lib.check(_bind().tb_decoder_set_attention_cap(self._h, int(cap)))

    # -- stepping -----------------------------------------------------------

    def _step(self, token_id: int, offset: int, want_logits: bool):
        out = np.empty(self.vocab_size, np.float32) if want_logits else None
        am = C.c_int64()
        _lib.check(_bind().tb_decoder_step(self._h, int(token_id), int(offset),
                                           out.ctypes.data if want_logits else None,
                                           C.byref(am)))
        return out, int(am.value)

    def decode_step(self, token_id: int, offset: int):
        """Logits of one step as a float32 tensor [1, vocab] (decoder.rs:729-750)."""
        import torch
        out, _ = self._step(token_id, offset, True)
        return torch.from_numpy(out).reshape(1, -1)

    def step(self, token_id: int, offset: int) -> List[float]:
        out, _ = self._step(token_id, offset, True)
        return out.tolist()

    def decode_and_sample(self, token_id: int, offset: int, temperature: float = 0.7,
                          top_k: int = 40, repetition_penalty: float = 1.0,
                          recent_tokens: Optional[Sequence[int]] = None,
                          top_p: float = 1.0) -> int:
        rec = np.asarray(list(recent_tokens or []), dtype=np.int64)
        out = C.c_int64()
        _lib.check(_bind().tb_decoder_decode_and_sample(
            self._h, int(token_id), int(offset), float(temperature), int(top_k),
            float(repetition_penalty), rec.ctypes.data if rec.size else None, rec.size,
            float(top_p), C.byref(out)))
        return int(out.value)

    def generate_loop(self, first_token: int, seq_len: int, max_new_tokens: int,
                      temperature: float = 0.7, top_k: int = 40,
                      repetition_penalty: float = 1.0, top_p: float = 1.0,
                      eos_token_id: Optional[int] = None,
                      recent_seed: Optional[Sequence[int]] = None) -> Tuple[List[int], int]:
        """Whole decode loop in one call (decoder.rs:788-832).  Sampling runs on
        the device for any top_k (see tb_decoder_generate_sampled)."""
        toks = np.empty(max(int(max_new_tokens), 1), np.int64)
        n, sl = C.c_int64(), C.c_int64()
        eos = -1 if eos_token_id is None else int(eos_token_id)
        greedy = not np.isfinite(temperature) or temperature <= 0 or top_k == 1
        if greedy and repetition_penalty <= 1.0:
            _lib.check(_bind().tb_decoder_generate(
                self._h, int(first_token), int(seq_len), int(max_new_tokens), eos,
                toks.ctypes.data, C.byref(n), C.byref(sl)))
        else:
            seed_ids = np.asarray(list(recent_seed or []), dtype=np.int64)
            _lib.check(_bind().tb_decoder_generate_sampled(
                self._h, int(first_token), int(seq_len), int(max_new_tokens), float(temperature),
                int(top_k), float(repetition_penalty), float(top_p), eos,
                seed_ids.ctypes.data if seed_ids.size else None, seed_ids.size,
                toks.ctypes.data, C.byref(n), C.byref(sl)))
        return toks[:n.value].tolist(), int(sl.value)

    def prefill_tokens(self, tokens: Sequence[int], start_offset: int) -> int:
        arr = np.asarray(list(tokens), dtype=np.int64)
        off = C.c_int64()
        _lib.check(_bind().tb_decoder_prefill(self._h, arr.ctypes.data if arr.size else None,
                                              arr.size, int(start_offset), C.byref(off)))
        return int(off.value)

    def prefill(self, tokens: Sequence[int]) -> List[float]:
        if len(tokens) == 0:
            raise ValueError("empty prefill")
        if len(tokens) > self.max_seq_len:
            raise ValueError("prefill exceeds max_seq_len")
        self.prefill_tokens(tokens, 0)
        return self.get_logits()

    def verify_tokens(self, start_offset: int, tokens: Sequence[int]) -> List[List[float]]:
        """Logits of every position (decoder.rs:565-581); INT4 decoders run the
        positions as one batched forward."""
        return self._verify(start_offset, tokens).tolist()

    def _verify(self, start_offset: int, tokens: Sequence[int]) -> np.ndarray:
        if start_offset + len(tokens) > self.max_seq_len:
            raise ValueError("verify exceeds max_seq_len")
        arr = np.asarray(list(tokens), dtype=np.int64)
        out = np.empty((arr.size, self.vocab_size), np.float32)
        _lib.check(_bind().tb_decoder_verify(self._h, int(start_offset),
                                             arr.ctypes.data if arr.size else None, arr.size,
                                             out.ctypes.data if arr.size else None))
        return out

    def speculative_accept(self, offset: int, draft_tokens: Sequence[int],
                           draft_probs: Sequence[float], temperature: float = 1.0,
                           top_p: float = 1.0) -> Tuple[int, int]:
        """(accepted, bonus) of the reference's speculative step (decoder.rs:588-727)."""
        arr = np.asarray(list(draft_tokens), dtype=np.int64)
        probs = np.ascontiguousarray(np.asarray(draft_probs, dtype=np.float32).reshape(-1))
        if arr.size and probs.size != arr.size * self.vocab_size:
            raise ValueError("draft_probs must be K×V row-major")
        a, b = C.c_int64(), C.c_int64()
        _lib.check(_bind().tb_decoder_speculative_accept(
            self._h, int(offset), arr.ctypes.data if arr.size else None, arr.size,
            probs.ctypes.data if probs.size else None, float(temperature), float(top_p),
            C.byref(a), C.byref(b)))
        return int(a.value), int(b.value)

    # -- KV cache -------------------------------------------------------------

    def reset_kv_cache(self) -> None:
        _lib.check(_bind().tb_decoder_reset_kv(self._h))

    def copy_kv_cache_from_tensors(self, k_tensors, v_tensors, seq_len: int) -> None:
        """Per-layer [.., kv_heads, src_max, head_dim] f32 tensors (decoder.rs:479-523)."""
        L = _bind()
        for li in range(min(self.num_layers, len(k_tensors))):
            shp = tuple(k_tensors[li].shape)
            if len(shp) < 2 or shp[-1] != self.head_dim or tuple(v_tensors[li].shape) != shp:
                raise _lib.UnsupportedOpError(
                    f"{_lib.UNSUPPORTED_MARKER} layer {li} KV tensors must be "
                    f"[.., {self.num_kv_heads}, src_max, {self.head_dim}], got {list(shp)} / "
                    f"{list(v_tensors[li].shape)}")
            src_max = int(shp[-2])
            n = self.num_kv_heads * src_max * self.head_dim
            kp, kk, _ = _as_buffer(k_tensors[li], np.float32, n, f"layer {li} k")
            vp, vk, _ = _as_buffer(v_tensors[li], np.float32, n, f"layer {li} v")
            _lib.check(L.tb_decoder_copy_kv(self._h, li, kp, vp, src_max, int(seq_len)))
            del kk, vk

    def kv_len(self) -> int:
        out = C.c_int64()
        _lib.check(_bind().tb_decoder_kv_len(self._h, C.byref(out)))
        return int(out.value)

    def get_logits(self) -> List[float]:
        out = np.empty(self.vocab_size, np.float32)
        _lib.check(_bind().tb_decoder_get_logits(self._h, out.ctypes.data))
        return out.tolist()

    def set_seed(self, seed: int) -> None:
        _lib.check(_bind().tb_decoder_set_seed(self._h, int(seed) & (2 ** 64 - 1)))

    def time_greedy(self, first_token: int, offset: int, n_steps: int) -> float:
        """Milliseconds for n_steps device-driven greedy steps (benchmark helper)."""
        ms = C.c_float()
        _lib.check(_bind().tb_decoder_time_greedy(self._h, int(first_token), int(offset),
                                                  int(n_steps), C.byref(ms)))
        return float(ms.value)

    def close(self) -> None:
        if self._h:
            _bind().tb_decoder_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def decoder_from_weights(w: dict, cfg: dict, group_size: int = 32,
                         max_seq_len: int = 2048) -> RustQwenDecoder:
    """RustQwenDecoder from a synthetic weight dict (torchburn_amd.synth.decoder_weights)."""
    layers = []
    for lw in w["layers"]:
        caps = [lw["in_norm"], lw["qkv_w"], lw["qkv_s"], lw["o_w"], lw["o_s"], lw["post_norm"],
                lw["gate_w"], lw["gate_s"], lw["up_w"], lw["up_s"], lw["down_w"], lw["down_s"]]
        if lw.get("qkv_b") is not None:
            caps.append(lw["qkv_b"])
        layers.append(caps)
    return RustQwenDecoder(w["embed"], layers, w["final_norm"], w["lm_head_w"], w["lm_head_s"],
                           cfg["num_layers"], cfg["hidden"], cfg["intermediate"],
                           cfg["num_heads"], cfg["num_kv_heads"], cfg["head_dim"], group_size,
                           cfg["eps"], max_seq_len, cfg["rope_theta"])


def create_rust_qwen_decoder(model: Any, max_seq_len: int = 4096,
                             group_size: Optional[int] = None) -> RustQwenDecoder:
    """From a quantized model with the reference's module layout
    (python/torchburn/quantization.py:575-647): embed_tokens, layers[i].
    {input_layernorm, self_attn.{qkv_proj,o_proj}, post_attention_layernorm,
    mlp.{gate,up,down}_proj}, norm, lm_head (QuantizedLinear or nn.Linear)."""
    layers = []
    for layer in model.layers:
        at, mlp = layer.self_attn, layer.mlp
        caps = [layer.input_layernorm.weight, at.qkv_proj.qweight, at.qkv_proj.scales,
                at.o_proj.qweight, at.o_proj.scales, layer.post_attention_layernorm.weight,
                mlp.gate_proj.qweight, mlp.gate_proj.scales, mlp.up_proj.qweight,
                mlp.up_proj.scales, mlp.down_proj.qweight, mlp.down_proj.scales]
        if getattr(at.qkv_proj, "bias", None) is not None:
            caps.append(at.qkv_proj.bias)
        layers.append([c.detach().float() if c.dtype.is_floating_point else c.detach()
                       for c in caps])
    cfg = model.config
    lm = model.lm_head
    if hasattr(lm, "qweight"):
        lm_w, lm_s = lm.qweight.detach(), lm.scales.detach().float()
    else:
        lm_w, lm_s = lm.weight.detach().float(), None
    gs = group_size or getattr(model.layers[0].mlp.gate_proj, "group_size", 64)
    return RustQwenDecoder(model.embed_tokens.weight.detach().float(), layers,
                           model.norm.weight.detach().float(), lm_w, lm_s, len(model.layers),
                           cfg.hidden_size, cfg.intermediate_size, cfg.num_attention_heads,
                           cfg.num_key_value_heads, cfg.head_dim, gs, cfg.rms_norm_eps,
                           max_seq_len, cfg.rope_theta)
