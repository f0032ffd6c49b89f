// Device-side range coder: one lane owns one independent stream.
//
// Bit-exact with the spec krunch_ac/cpu_reference.py:91-234: 32-bit
// low/high, E1/E2/E3 renormalisation, pending (E3) bits emitted as
// complements after the next decided bit, MSB-first packing, a flush of one
// bit plus pending+1 complements, and zero bits read past the end of a
// stream. Interval arithmetic in 64 bits as in encode_kernel.cu:112-116.
#pragma once
#include "kr_common.h"

// MSB-first bit writer over one stream's bytes. Bits already present in the
// partial byte at the starting offset are kept (the buffer is zero-filled by
// the caller, as in the reference's contract), completed bytes are stored
// whole, writes at or past `cap` are dropped and counted in `overflow`.
struct kr_bit_sink {
    uint8_t* buf;
    uint32_t byte;
    uint32_t cur;
    uint32_t nb;
    uint32_t cap;
    uint32_t overflow;

    __device__ void open(uint8_t* b, uint32_t bitpos, uint32_t capacity) {
        buf = b;
        byte = bitpos >> 3;
        nb = bitpos & 7u;
        cap = capacity;
        overflow = 0;
        cur = 0;
        if (nb) cur = (byte < cap ? (uint32_t)buf[byte] : 0u) & ((0xFF00u >> nb) & 0xFFu);
    }
    __device__ void emit_byte() {
        if (byte < cap) buf[byte] = (uint8_t)cur;
        else overflow = 1;
        byte++;
        cur = 0;
        nb = 0;
    }
    __device__ void put(uint32_t bit) {
        cur |= bit << (7u - nb);
        if (++nb == 8u) emit_byte();
    }
    __device__ void put_run(uint32_t bit, uint32_t n) {
        while (n && nb) { put(bit); n--; }
        const uint32_t fill = bit ? 0xFFu : 0u;
        while (n >= 8u) { cur = fill; emit_byte(); n -= 8u; }
        while (n) { put(bit); n--; }
    }
    // Stores the trailing partial byte; returns the new bit offset.
    __device__ uint32_t close() {
        if (nb) {
            if (byte < cap) buf[byte] = (uint8_t)cur;
            else overflow = 1;
        }
        return byte * 8u + nb;
    }
};

// MSB-first bit reader; bytes at index >= limit read as zero.
struct kr_bit_source {
    const uint8_t* buf;
    uint32_t limit;
    uint32_t pos;
    __device__ uint32_t get() {
        const uint32_t byte = pos >> 3;
        const uint32_t b = byte < limit ? (uint32_t)buf[byte] : 0u;
        const uint32_t bit = (b >> (7u - (pos & 7u))) & 1u;
        pos++;
        return bit;
    }
};

// The next 64 bits of a stream from bit `pos`, fetched with eight independent
// byte loads (bytes at index >= limit read as zero). One decode step consumes
// at most 26 bits (the narrowed interval is at least 2^6 wide and doubles per
// bit), so a window taken before the step covers it; reads beyond the window
// fall back to the byte reader.
struct kr_bit_window {
    const uint8_t* buf;
    uint32_t limit;
    uint32_t base;     // bit index of the window's first bit (multiple of 8)
    uint32_t pos;
    uint64_t w;
    __device__ void open(const uint8_t* b, uint32_t lim, uint32_t bitpos) {
        buf = b;
        limit = lim;
        pos = bitpos;
        base = bitpos & ~7u;
        const uint32_t byte = bitpos >> 3;
        w = 0;
        if (limit == 0) return;
        // eight loads at in-bounds (clamped) addresses, issued together; bytes
        // past the limit read as zero
        uint32_t v[8];
        #pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t bi = byte + (uint32_t)i;
            v[i] = buf[bi < limit ? bi : limit - 1u];
        }
        #pragma unroll
        for (int i = 0; i < 8; i++)
            if (byte + (uint32_t)i < limit) w |= (uint64_t)v[i] << (56 - 8 * i);
    }
    __device__ uint32_t get() {
        const uint32_t off = pos - base;
        uint32_t bit;
        if (off < 64u) {
            bit = (uint32_t)(w >> (63u - off)) & 1u;
        } else {
            const uint32_t byte = pos >> 3;
            const uint32_t b = byte < limit ? (uint32_t)buf[byte] : 0u;
            bit = (b >> (7u - (pos & 7u))) & 1u;
        }
        pos++;
        return bit;
    }
};

// Narrow [low, high] to the symbol's cumulative range [c_lo, c_hi) of 2^prec.
__device__ __forceinline__ void kr_rc_narrow(uint32_t& low, uint32_t& high, uint32_t c_lo,
                                             uint32_t c_hi, int prec) {
    const uint64_t span = (uint64_t)(high - low) + 1ull;
    const uint32_t nh = low + (uint32_t)((span * (uint64_t)c_hi) >> prec) - 1u;
    const uint32_t nl = low + (uint32_t)((span * (uint64_t)c_lo) >> prec);
    low = nl;
    high = nh;
}

__device__ __forceinline__ void kr_rc_encode(uint32_t& low, uint32_t& high, uint32_t& pending,
                                             uint32_t c_lo, uint32_t c_hi, int prec,
                                             kr_bit_sink& sink) {
    kr_rc_narrow(low, high, c_lo, c_hi, prec);
    for (;;) {
        if (high < KR_RC_HALF) {
            sink.put(0u);
            sink.put_run(1u, pending);
            pending = 0;
            low <<= 1;
            high = (high << 1) | 1u;
        } else if (low >= KR_RC_HALF) {
            sink.put(1u);
            sink.put_run(0u, pending);
            pending = 0;
            low = (low - KR_RC_HALF) << 1;
            high = ((high - KR_RC_HALF) << 1) | 1u;
        } else if (low >= KR_RC_QUARTER && high < KR_RC_3QUARTER) {
            pending++;
            low = (low - KR_RC_QUARTER) << 1;
            high = ((high - KR_RC_QUARTER) << 1) | 1u;
        } else {
            break;
        }
    }
}

__device__ __forceinline__ void kr_rc_flush(uint32_t low, uint32_t pending, kr_bit_sink& sink) {
    const uint32_t bit = (low < KR_RC_QUARTER) ? 0u : 1u;
    sink.put(bit);
    sink.put_run(1u - bit, pending + 1u);
}

// Decoder target: floor(((value - low + 1) * 2^prec - 1) / (high - low + 1)).
__device__ __forceinline__ uint32_t kr_rc_target(uint32_t low, uint32_t high, uint32_t value,
                                                 int prec) {
    const uint64_t span = (uint64_t)(high - low) + 1ull;
    const uint64_t off = (uint64_t)(value - low) + 1ull;
    return (uint32_t)(((off << prec) - 1ull) / span);
}

template <class Source>
__device__ __forceinline__ void kr_rc_consume(uint32_t& low, uint32_t& high, uint32_t& value,
                                              uint32_t c_lo, uint32_t c_hi, int prec,
                                              Source& src) {
    kr_rc_narrow(low, high, c_lo, c_hi, prec);
    for (;;) {
        uint32_t shift;
        if (high < KR_RC_HALF) shift = 0u;
        else if (low >= KR_RC_HALF) shift = KR_RC_HALF;
        else if (low >= KR_RC_QUARTER && high < KR_RC_3QUARTER) shift = KR_RC_QUARTER;
        else break;
        low = (low - shift) << 1;
        high = ((high - shift) << 1) | 1u;
        value = ((value - shift) << 1) | src.get();
    }
}
