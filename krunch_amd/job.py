"""Worker job runner for distributed compress / decompress (the role of
krunch/job.py:1-255), for local paths and file:// URLs.

The env-var contract is the reference's (job.py:18-39):

  KRUNCH_MODE          compress | decompress | finalize
  KRUNCH_INPUT_URL     source (compress: raw bytes; decompress: a .krunch blob)
  KRUNCH_OUTPUT_URL    final output; parts go to <KRUNCH_OUTPUT_URL>.parts/part-NNNNNN
  KRUNCH_PART_INDEX    0-based index of this worker (compress, decompress)
  KRUNCH_PART_COUNT    number of workers
  KRUNCH_INPUT_LEN     total input bytes (compress, finalize of compress)
  KRUNCH_FINALIZE_OF   compress | decompress (finalize)

A compress worker takes the byte range [start, end) that every worker
derives from KRUNCH_INPUT_LEN alone: the boundaries fall on multiples of the
whole input's chunk size, so the ranges need no coordination and each part
is cut into chunks of that size. It writes a .krunch blob of its slice. A decompress
worker takes a contiguous run of ceil(n_chunks / part_count) chunks and
writes their raw bytes. Finalize joins the compress parts under one master
header (flags 0x01: no whole-file CRC, as the reference's assembled blobs)
or concatenates the raw parts, then deletes the parts.

The model comes from $KRUNCH_WEIGHTS / $KRUNCH_TOKENIZER (else the synthetic
model and the byte tokenizer); $KRUNCH_W8A8=1 selects the int8 codec for
compress, and decompress takes the codec from the blob. Object-storage URLs
(s3://, http://) are outside this build and are rejected with an error.
"""
from __future__ import annotations

import logging
import os
import struct
import sys
import zlib
from typing import Callable, Mapping, Optional, Tuple

from krunch_amd import chunking
from krunch_amd.inference import (HEADER_SIZE, MODEL_ID_W8A8, InferenceEngine, decode_header,
                                  encode_header)

logger = logging.getLogger("krunch_amd.job")

FLAG_NO_CRC = 0x01


def _local(url: str) -> str:
    if url.startswith("file://"):
        return url[len("file://"):]
    if "://" in url:
        raise ValueError(f"unsupported URL {url!r}: only local paths and file:// are handled here")
    return url


def _read_range(url: str, start: int, end: int) -> bytes:
    with open(_local(url), "rb") as f:
        f.seek(start)
        return f.read(max(0, end - start))


def _read_all(url: str) -> bytes:
    with open(_local(url), "rb") as f:
        return f.read()


def _write(url: str, data: bytes) -> None:
    path = _local(url)
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    tmp = path + ".tmp"
    with open(tmp, "wb") as f:
        f.write(data)
    os.replace(tmp, path)


def part_url(output_url: str, index: int) -> str:
    """<output>.parts/part-NNNNNN (job.py:237-240)."""
    return f"{output_url.rstrip('/')}.parts/part-{index:06d}"


def byte_range(part_index: int, part_count: int, total_size: int) -> Tuple[int, int]:
    """[start, end) of a compress worker's slice (job.py:243-255): every part
    but the last covers the same whole number of chunks (at least one), the
    last takes the rest; a part past the input is empty."""
    if part_count < 1 or not 0 <= part_index < part_count:
        raise ValueError(f"bad part {part_index} of {part_count}")
    chunk = chunking.compute_chunk_size(total_size)
    per_part = max(chunk, total_size // part_count // chunk * chunk)
    start = min(part_index * per_part, total_size)
    end = total_size if part_index == part_count - 1 else min(start + per_part, total_size)
    return start, end


def chunk_range(part_index: int, part_count: int, n_chunks: int) -> Tuple[int, int]:
    """[lo, hi) of a decompress worker's chunks (job.py:150-153)."""
    if part_count < 1 or not 0 <= part_index < part_count:
        raise ValueError(f"bad part {part_index} of {part_count}")
    per = (n_chunks + part_count - 1) // part_count
    lo = min(part_index * per, n_chunks)
    return lo, min(lo + per, n_chunks)


def load_engine(w8a8: bool) -> InferenceEngine:
    return InferenceEngine().load(os.environ.get("KRUNCH_WEIGHTS") or None,
                                  tokenizer_path=os.environ.get("KRUNCH_TOKENIZER") or None,
                                  w8a8=w8a8)


def compress_part(env: Mapping[str, str], load: Callable[[bool], object] = load_engine) -> None:
    src, dst = env["KRUNCH_INPUT_URL"], env["KRUNCH_OUTPUT_URL"]
    total = int(env["KRUNCH_INPUT_LEN"])
    count, index = int(env["KRUNCH_PART_COUNT"]), int(env["KRUNCH_PART_INDEX"])
    start, end = byte_range(index, count, total)
    raw = _read_range(src, start, end)
    if len(raw) != end - start:
        raise ValueError(f"input shorter than KRUNCH_INPUT_LEN: read {len(raw)} of [{start}, {end})")
    eng = load(env.get("KRUNCH_W8A8", "0") == "1")
    # the whole input's chunk size, so the part's chunks line up with the ranges
    entries, n = chunking.compress_all(raw, eng.compress_chunk,
                                       neural_batch_fn=eng.compress_chunks_batched,
                                       total_size=total)
    blob = encode_header(len(raw), n, zlib.crc32(raw) & 0xFFFFFFFF, model_id=eng.model_id,
                         tokenizer_id=eng.tokenizer_id) + b"".join(entries)
    _write(part_url(dst, index), blob)
    logger.info("compress part %d/%d: bytes [%d, %d) -> %d bytes, %d chunks",
                index, count, start, end, len(blob), n)


def decompress_part(env: Mapping[str, str], load: Callable[[bool], object] = load_engine) -> None:
    src, dst = env["KRUNCH_INPUT_URL"], env["KRUNCH_OUTPUT_URL"]
    count, index = int(env["KRUNCH_PART_COUNT"]), int(env["KRUNCH_PART_INDEX"])
    blob = _read_all(src)
    hdr = decode_header(blob)
    chunks = chunking.parse_entries(blob[HEADER_SIZE:], hdr["n_chunks"])
    lo, hi = chunk_range(index, count, len(chunks))
    mine = b"".join(struct.pack(">II", ol, len(enc)) + enc for ol, enc in chunks[lo:hi])
    raw = b""
    if hi > lo:
        eng = load(hdr["model_id"] == MODEL_ID_W8A8)
        if hdr["model_id"] != eng.model_id or hdr["tokenizer_id"] != eng.tokenizer_id:
            raise ValueError(f"blob codec (model {hdr['model_id']}, tokenizer {hdr['tokenizer_id']}) "
                             f"!= loaded ({eng.model_id}, {eng.tokenizer_id})")
        raw = chunking.decompress_all(mine, hi - lo, eng.decompress_chunk,
                                      neural_batch_fn=eng.decompress_chunks_batched)
    _write(part_url(dst, index), raw)
    logger.info("decompress part %d/%d: chunks [%d, %d) -> %d bytes", index, count, lo, hi, len(raw))


def finalize(env: Mapping[str, str]) -> None:
    dst = env["KRUNCH_OUTPUT_URL"]
    count = int(env["KRUNCH_PART_COUNT"])
    of = env.get("KRUNCH_FINALIZE_OF", "compress").lower()
    parts = [_read_all(part_url(dst, i)) for i in range(count)]
    if of == "compress":
        heads = [decode_header(p) for p in parts]
        codecs = {(h["model_id"], h["tokenizer_id"]) for h in heads}
        if len(codecs) != 1:
            raise ValueError(f"parts were compressed with different codecs: {sorted(codecs)}")
        model_id, tokenizer_id = codecs.pop()
        original_len = int(env["KRUNCH_INPUT_LEN"])
        if sum(h["original_len"] for h in heads) != original_len:
            raise ValueError("parts do not add up to KRUNCH_INPUT_LEN")
        out = encode_header(original_len, sum(h["n_chunks"] for h in heads), 0, flags=FLAG_NO_CRC,
                            model_id=model_id, tokenizer_id=tokenizer_id) + \
            b"".join(p[HEADER_SIZE:] for p in parts)
    elif of == "decompress":
        out = b"".join(parts)
    else:
        raise ValueError(f"KRUNCH_FINALIZE_OF must be compress or decompress, got {of!r}")
    _write(dst, out)
    for i in range(count):
        try:
            os.remove(_local(part_url(dst, i)))
        except OSError as e:
            logger.warning("part cleanup failed: %s", e)
    try:
        os.rmdir(_local(dst.rstrip("/") + ".parts"))
    except OSError:
        pass
    logger.info("finalize %s: %d parts -> %d bytes", of, count, len(out))


def run(env: Optional[Mapping[str, str]] = None,
        load: Callable[[bool], object] = load_engine) -> int:
    """Dispatch on KRUNCH_MODE; 0 on success, 1 on a bad contract or input."""
    env = os.environ if env is None else env
    mode = env.get("KRUNCH_MODE", "").lower()
    try:
        if mode == "compress":
            compress_part(env, load)
        elif mode == "decompress":
            decompress_part(env, load)
        elif mode == "finalize":
            finalize(env)
        else:
            raise ValueError(f"KRUNCH_MODE must be compress, decompress or finalize, got {mode!r}")
    except (KeyError, ValueError, OSError) as e:
        logger.error("job failed: %s", e)
        return 1
    return 0


if __name__ == "__main__":
    logging.basicConfig(level=logging.INFO, format="%(asctime)s %(levelname)s %(message)s",
                        stream=sys.stderr)
    sys.exit(run())
