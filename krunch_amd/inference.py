"""Drop-in for the codec engine of `krunch.inference` (`krunch/inference.py`).

Kept from the reference: the blob header (`encode_header`/`decode_header`,
format ">4sBIIIHHQII", 37 bytes; inference.py:47-83), BOS = 0, the per-chunk
mini-header ">II" (orig_len, n_tokens) followed by the range-coded bits
(inference.py:357-360), and the engine methods `load`, `compress_chunk`,
`decompress_chunk`, `compress_chunks_batched`, `decompress_chunks_batched`.

The hot path is token level: `compress_tokens_batched` runs B chunks through
packed windows of KRUNCH_FORWARD_BATCH (1024) tokens with RNN and coder state
carried across windows (inference.py:311-338, generalised from one chunk to B
chunks per call); `decompress_tokens_batched` decodes B chunks in lockstep,
one token per stream per step, with the CDF search and range decode fused on
the GPU and the whole step replayed from one HIP graph (inference.py:363-443).
Byte-level methods tokenize with a `tokenizers` JSON when one is loaded,
else with the byte tokenizer (krunch_amd/tokenizer.py); `compress` /
`decompress` write and read the `.krunch` container (cli.py:49-118,
chunking.py) with CRC32, length and codec checks.
"""
from __future__ import annotations

import os
import struct
import zlib
from typing import List, Optional, Sequence

import numpy as np
import torch

from krunch_amd import _lib, cpp_path
from krunch_amd.model import State

BLOB_MAGIC = b"KRNC"
BLOB_VERSION = 1
MODEL_ID = 1            # fp16 codec
MODEL_ID_W8A8 = 2       # w8a8 codec (int8 layer products; a different bitstream)
TOKENIZER_ID = 1
HEADER_FMT = ">4sBIIIHHQII"
HEADER_SIZE = struct.calcsize(HEADER_FMT)
BOS_TOKEN = 0
CDF_PRECISION = 24


DEFAULT_STREAM_BATCH = cpp_path.DEFAULT_STREAM_BATCH

# Rows per head GEMM + CDF block of a compress window: the logits buffer
# holds this many rows (8192 x 50280 fp16 = 824 MB of the 288 GB). Measured on
# MI355X (bench window, A B A B): compress 8,804 / 8,793 KB/s at 4,096 rows,
# 8,838 / 8,833 at 8,192, 8,748 / 8,680 at 16,384.
HEAD_ROWS = 8192

# Largest coder buffer of one lockstep call, in bytes. Stream offsets into it
# are int32 and its length is a uint32 in the C ABI (the reference's
# base_byte_offsets are int32 too, encode_kernel.cu:148-197), so a call whose
# concatenated bitstreams would exceed 2^31 - 1 bytes is split into several.
MAX_CALL_BYTES = (1 << 31) - 1


def coder_stream_cap(n_tokens: int) -> int:
    """Output bytes reserved per stream for n_tokens symbols. A symbol costs at
    most CDF_PRECISION + 2 bits plus pending bits that the same budget covers;
    4 bytes per token + 64 bounds every stream (an overflow raises)."""
    return int(4 * n_tokens + 64)


def split_by_bytes(sizes: Sequence[int], limit: int) -> List[range]:
    """Consecutive index ranges whose byte sizes sum to <= limit each (one
    item per range at least; an item larger than limit is an error)."""
    out, start, acc = [], 0, 0
    for i, n in enumerate(sizes):
        if n > limit:
            raise ValueError(f"one stream needs {n} coder bytes > the per-call limit {limit}")
        if acc + n > limit and i > start:
            out.append(range(start, i))
            start, acc = i, 0
        acc += n
    if len(sizes) > start:
        out.append(range(start, len(sizes)))
    return out


compute_decompress_batch = cpp_path.compute_decompress_batch


def compute_compress_batch(n_chunks: int = -1, default: int = DEFAULT_STREAM_BATCH) -> int:
    """Streams compressed in one packed call; $KRUNCH_COMPRESS_BATCH overrides."""
    return cpp_path.env_batch("KRUNCH_COMPRESS_BATCH", n_chunks, default)


def encode_header(original_len: int, n_chunks: int, crc32: int, adapter_id: int = 0,
                  adapter_version: int = 0, flags: int = 0, model_id: int = MODEL_ID,
                  tokenizer_id: int = TOKENIZER_ID) -> bytes:
    return struct.pack(HEADER_FMT, BLOB_MAGIC, BLOB_VERSION, model_id, tokenizer_id, adapter_id,
                       adapter_version, flags, original_len, n_chunks, crc32)


def decode_header(data: bytes) -> dict:
    if len(data) < HEADER_SIZE:
        raise ValueError(f"blob too short: {len(data)} < {HEADER_SIZE}")
    magic, bv, mid, tid, aid, av, flags, orig_len, n_chunks, crc = struct.unpack(
        HEADER_FMT, data[:HEADER_SIZE])
    if magic != BLOB_MAGIC:
        raise ValueError(f"bad magic: {magic!r}")
    return {"blob_version": bv, "model_id": mid, "tokenizer_id": tid, "adapter_id": aid,
            "adapter_version": av, "flags": flags, "original_len": orig_len,
            "n_chunks": n_chunks, "crc32": crc}


class InferenceEngine:
    def __init__(self):
        self._weights = None
        self._tokenizer = None
        self._ready = False
        self.window = int(os.environ.get("KRUNCH_FORWARD_BATCH", "1024"))
        self.use_graph = os.environ.get("KRUNCH_HIP_GRAPH", "1") == "1"
        # lockstep streams may be split into concurrent groups (graph branches); one
        # group measured fastest on MI355X (branches of one graph do not overlap)
        self.decode_groups = int(os.environ.get("KRUNCH_DECODE_GROUPS", "1"))
        self.model_id = MODEL_ID
        self.max_call_bytes = MAX_CALL_BYTES

    # ------------------------------------------------------------------ setup
    def load(self, weights: Optional[dict] = None, tokenizer_path: Optional[str] = None,
             device: str = "cuda", w8a8: bool = False, rescale: bool = True):
        """Prepare weights and an optional tokenizer. `weights` is a dict in
        the engine layout (rwkv-package keys, [in, out] matrices, raw
        time_decay), a path to an RWKV-4 `.pth` / `.safetensors` checkpoint
        (converted by krunch_amd.weights.load_rwkv4), or None for the
        synthetic RWKV-4-169M-shaped model (seed 0). w8a8=True selects the
        int8 codec (model_id 2): its streams decode only with the int8 codec.
        rescale applies to checkpoint paths only (krunch_amd.weights): True,
        the default, computes what the reference codec computes on that
        checkpoint."""
        if weights is None:
            from krunch_amd.synthetic import make_weights
            weights = make_weights()
        elif isinstance(weights, (str, os.PathLike)):
            from krunch_amd.weights import load_rwkv4
            weights = load_rwkv4(weights, rescale=rescale)
        self._weights = cpp_path.init_weights(weights, device, w8a8=w8a8)
        self.model_id = MODEL_ID_W8A8 if w8a8 else MODEL_ID
        from krunch_amd.tokenizer import load_tokenizer
        self._tokenizer = load_tokenizer(tokenizer_path)
        self._ready = True
        return self

    @property
    def tokenizer_id(self) -> int:
        """1 for a tokenizers JSON (the reference's id), 0 for the byte tokenizer."""
        return self._tokenizer.tokenizer_id if self._tokenizer is not None else TOKENIZER_ID

    @property
    def ready(self) -> bool:
        return self._ready

    @property
    def weights(self):
        return self._weights

    # -------------------------------------------------------------- compress
    def compress_tokens_batched(self, token_streams: Sequence[np.ndarray],
                                orig_lens: Optional[Sequence[int]] = None) -> List[bytes]:
        """B token streams -> B chunk payloads (">II" mini-header + bits), in
        calls of at most compute_compress_batch() streams."""
        assert self._ready, "call load() first"
        B = len(token_streams)
        if B == 0:
            return []
        lens = np.array([len(t) for t in token_streams], dtype=np.int64)
        if (lens < 1).any():
            raise ValueError("chunk has no tokens")
        Tmax = int(lens.max())
        per_cap = coder_stream_cap(Tmax)
        # streams per call: the batch size, and a coder buffer of <= max_call_bytes
        cap = min(compute_compress_batch(B), max(1, self.max_call_bytes // per_cap))
        if per_cap > self.max_call_bytes:
            raise ValueError(f"a {Tmax}-token stream needs {per_cap} coder bytes > the "
                             f"per-call limit {self.max_call_bytes}")
        if B > cap:
            res: List[bytes] = []
            for i in range(0, B, cap):
                res += self.compress_tokens_batched(
                    token_streams[i:i + cap], None if orig_lens is None else orig_lens[i:i + cap])
            return res
        W = self._weights
        P = W["prepared"]
        dev = P.device
        tok = np.zeros((B, Tmax), dtype=np.int32)
        for b, t in enumerate(token_streams):
            tok[b, :len(t)] = np.asarray(t, dtype=np.int32)
        if tok.min() < 0 or tok.max() >= P.V:
            raise ValueError(f"token id out of range [0, {P.V})")
        inp = np.zeros_like(tok)
        inp[:, 0] = BOS_TOKEN
        inp[:, 1:] = tok[:, :-1]
        tok_d = torch.from_numpy(tok).to(dev)
        inp_d = torch.from_numpy(inp).to(dev)

        out = torch.zeros(B * per_cap, dtype=torch.uint8, device=dev)
        out_cap = _lib.u32(out.numel(), "coder buffer bytes")
        base = torch.arange(B, dtype=torch.int32, device=dev) * per_cap
        ac = torch.zeros((B, 4), dtype=torch.int64)
        ac[:, 1] = 0xFFFFFFFF
        ac = ac.to(torch.uint32).to(dev).contiguous()
        err = torch.zeros(1, dtype=torch.uint32, device=dev)
        state = State(P.n_layer, B, P.C, dev)
        Tw = min(self.window, Tmax)
        M = B * Tw
        ws, nbytes = cpp_path.workspace(W, M)
        x = torch.empty((M, P.C), dtype=torch.float16, device=dev)
        head_rows = min(M, HEAD_ROWS)
        ld = cpp_path.logits_ld(P.V)
        logits = torch.empty((head_rows, ld), dtype=torch.float16, device=dev)
        lens_d = torch.from_numpy(lens.astype(np.int32)).to(dev)
        s = _lib.stream_ptr()
        # The range encoder (one lane per stream) of window w runs on its own
        # stream while window w+1's forward runs: the (cdf[s], cdf[s+1]) pairs
        # are double buffered, and the forward of window w+2 waits for the
        # encoder of window w before overwriting its buffer.
        main = torch.cuda.current_stream(dev)
        enc = torch.cuda.Stream(device=dev)
        pairs = [torch.empty((M, 2), dtype=torch.uint32, device=dev) for _ in range(2)]
        fwd_done = [torch.cuda.Event() for _ in range(2)]
        enc_done = [torch.cuda.Event() for _ in range(2)]
        windows = list(range(0, Tmax, Tw))
        n_valid = [(lens_d - w0).clamp(0, min(Tw, Tmax - w0)).to(torch.int32).contiguous()
                   for w0 in windows]
        for i, w0 in enumerate(windows):
            T = min(Tw, Tmax - w0)
            ids = inp_d[:, w0:w0 + T].contiguous()
            tgt = tok_d[:, w0:w0 + T].contiguous()
            buf = pairs[i % 2]
            if i >= 2:
                main.wait_event(enc_done[i % 2])
            _lib.call("kr_compress_window", P.ptr, ids.data_ptr(), tgt.data_ptr(), B, T, state.ptr,
                      x.data_ptr(), ws.data_ptr(), nbytes, logits.data_ptr(), ld, head_rows,
                      buf.data_ptr(), CDF_PRECISION, s)
            fwd_done[i % 2].record(main)
            enc.wait_event(fwd_done[i % 2])
            _lib.call("kr_encode_pairs_batched", buf.data_ptr(), T, T, n_valid[i].data_ptr(),
                      out.data_ptr(), out_cap, base.data_ptr(), ac.data_ptr(), B,
                      CDF_PRECISION, err.data_ptr(), enc.cuda_stream)
            enc_done[i % 2].record(enc)
        main.wait_stream(enc)
        _lib.call("kr_encode_finalize_batched", out.data_ptr(), out_cap, base.data_ptr(),
                  ac.data_ptr(), B, err.data_ptr(), s)
        if int(err.item()):
            raise RuntimeError("range coder output buffer overflow")
        bits = ac[:, 3].to(torch.int64).cpu().numpy()
        host = out.cpu().numpy()
        res = []
        for b in range(B):
            n = int((bits[b] + 7) // 8)
            ol = int(orig_lens[b]) if orig_lens is not None else 4 * int(lens[b])
            res.append(struct.pack(">II", ol, int(lens[b])) +
                       host[b * per_cap:b * per_cap + n].tobytes())
        return res

    # ------------------------------------------------------------ decompress
    def decompress_tokens_batched(self, encoded_chunks: Sequence[bytes]) -> List[np.ndarray]:
        """Chunk payloads -> token streams, decoded in lockstep in calls of at
        most compute_decompress_batch() streams."""
        assert self._ready, "call load() first"
        B = len(encoded_chunks)
        if B == 0:
            return []
        cap = compute_decompress_batch(B)
        # calls of <= cap streams whose concatenated bitstreams (+1 pad byte)
        # fit the int32 offsets / uint32 length of the decoder interface
        parts = [r for g in split_by_bytes([len(e) - 8 + 1 for e in encoded_chunks],
                                           self.max_call_bytes)
                 for r in (range(i, min(i + cap, g.stop)) for i in range(g.start, g.stop, cap))]
        if len(parts) > 1:
            res: List[np.ndarray] = []
            for r in parts:
                res += self.decompress_tokens_batched(encoded_chunks[r.start:r.stop])
            return res
        W = self._weights
        P = W["prepared"]
        dev = P.device
        n_tok, streams = [], []
        for enc in encoded_chunks:
            _, nt = struct.unpack(">II", enc[:8])
            n_tok.append(nt)
            streams.append(enc[8:])
        offs = np.cumsum([0] + [len(s) for s in streams])
        cat = np.frombuffer(b"".join(streams) + b"\0", dtype=np.uint8)
        inbuf = torch.from_numpy(cat.copy()).to(dev)
        in_len = _lib.u32(inbuf.numel(), "decoder input bytes")
        base = torch.from_numpy(offs[:-1].astype(np.int32)).to(dev)
        limits = torch.from_numpy(np.array([len(s) for s in streams], dtype=np.int32)).to(dev)
        ac = torch.empty((B, 4), dtype=torch.uint32, device=dev)
        s = _lib.stream_ptr()
        _lib.call("kr_decode_init_batched", inbuf.data_ptr(), in_len, base.data_ptr(),
                  limits.data_ptr(), ac.data_ptr(), B, s)
        Tmax = max(n_tok)
        state = State(P.n_layer, B, P.C, dev)
        syms = torch.full((B,), BOS_TOKEN, dtype=torch.int32, device=dev)
        tokens = torch.zeros((B, Tmax), dtype=torch.int32, device=dev)
        count = torch.zeros(B, dtype=torch.int32, device=dev)
        ntd = torch.tensor(n_tok, dtype=torch.int32, device=dev)
        x = torch.empty((B, P.C), dtype=torch.float16, device=dev)
        G = max(1, min(self.decode_groups, B))
        nbytes = _lib.lib().kr_decode_workspace_bytes(B, G, P.C, P.F)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        ld = cpp_path.logits_ld(P.V)
        logits = torch.empty((B, ld), dtype=torch.float16, device=dev)
        _lib.call("kr_decode_run", P.ptr, B, state.ptr, syms.data_ptr(), x.data_ptr(),
                  ws.data_ptr(), nbytes, logits.data_ptr(), ld, inbuf.data_ptr(), in_len,
                  base.data_ptr(), limits.data_ptr(), ac.data_ptr(), tokens.data_ptr(), Tmax,
                  count.data_ptr(), ntd.data_ptr(), CDF_PRECISION, Tmax, G,
                  1 if self.use_graph else 0, s)
        host = tokens.cpu().numpy()
        return [host[b, :n_tok[b]].copy() for b in range(B)]

    # ------------------------------------------------------------ byte level
    # inference.py:203-230,483-497,576-747: chunk bytes -> tokens -> payload
    # (`>II` orig_len, n_tokens + bits) and back, B chunks per batched call.
    def _need_tokenizer(self):
        if self._tokenizer is None:
            raise RuntimeError("call load() first")

    def compress_chunk(self, data: bytes) -> bytes:
        return self.compress_chunks_batched([data])[0]

    def compress_chunks_batched(self, chunks: Sequence[bytes]) -> List[bytes]:
        self._need_tokenizer()
        toks = [self._tokenizer.encode_bytes(c) for c in chunks]
        return self.compress_tokens_batched(toks, orig_lens=[len(c) for c in chunks])

    def decompress_chunk(self, encoded: bytes) -> bytes:
        return self.decompress_chunks_batched([encoded])[0]

    def decompress_chunks_batched(self, encoded_chunks: Sequence[bytes]) -> List[bytes]:
        self._need_tokenizer()
        toks = self.decompress_tokens_batched(encoded_chunks)
        out = []
        for enc, t in zip(encoded_chunks, toks):
            orig_len, _ = struct.unpack(">II", enc[:8])
            out.append(self._tokenizer.decode_bytes(t)[:orig_len])
        return out

    # ------------------------------------------------------------- container
    def compress(self, raw: bytes, chunk_size: Optional[int] = None) -> bytes:
        """bytes -> .krunch blob: header (model_id, tokenizer_id, length,
        chunk count, CRC32) + one `>II`(orig_len, comp_len) entry per chunk
        (cli.py:49-70, chunking.py:88-111); all chunks in one batched call."""
        from krunch_amd import chunking
        entries, n = chunking.compress_all(raw, self.compress_chunk,
                                           neural_batch_fn=self.compress_chunks_batched,
                                           chunk_size=chunk_size)
        crc = zlib.crc32(raw) & 0xFFFFFFFF
        return encode_header(len(raw), n, crc, model_id=self.model_id,
                             tokenizer_id=self.tokenizer_id) + b"".join(entries)

    def decompress(self, blob: bytes) -> bytes:
        """.krunch blob -> bytes, all chunks decoded in lockstep; checks the
        codec (model_id / tokenizer_id), the CRC32 unless flags bit 0 says
        there is none, and the length (cli.py:73-118)."""
        from krunch_amd import chunking
        hdr = decode_header(blob)
        if hdr["model_id"] != self.model_id:
            raise ValueError(f"blob model_id {hdr['model_id']} != loaded codec {self.model_id}")
        if hdr["tokenizer_id"] != self.tokenizer_id:
            raise ValueError(f"blob tokenizer_id {hdr['tokenizer_id']} != loaded {self.tokenizer_id}")
        raw = chunking.decompress_all(blob[HEADER_SIZE:], hdr["n_chunks"], self.decompress_chunk,
                                      neural_batch_fn=self.decompress_chunks_batched)
        if not hdr["flags"] & 0x01:
            actual = zlib.crc32(raw) & 0xFFFFFFFF
            if actual != hdr["crc32"]:
                raise ValueError(f"CRC32 mismatch: got {actual:#010x}, expected {hdr['crc32']:#010x}")
        if len(raw) != hdr["original_len"]:
            raise ValueError(f"length mismatch: got {len(raw)}, expected {hdr['original_len']}")
        return raw


engine = InferenceEngine()
