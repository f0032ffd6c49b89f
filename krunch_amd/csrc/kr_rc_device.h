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
// Bits gather in a 64-bit accumulator (MSB first) and leave four bytes at a
// time, so a run of n bits costs one or two shifts instead of n steps.
struct kr_bit_sink {
    uint8_t* buf;
    uint32_t byte;      // index of the byte the accumulator's top byte goes to
    uint64_t acc;       // pending bits, MSB-aligned
    uint32_t nacc;      // number of pending bits (< 32 between calls)
    uint32_t cap;
    uint32_t overflow;

    __device__ void open(uint8_t* b, uint32_t bitpos, uint32_t capacity) {
        buf = b;
        byte = bitpos >> 3;
        nacc = bitpos & 7u;
        cap = capacity;
        overflow = 0;
        acc = 0;
        if (nacc) {
            const uint32_t keep = (byte < cap ? (uint32_t)buf[byte] : 0u) & ((0xFF00u >> nacc) & 0xFFu);
            acc = (uint64_t)keep << 56;
        }
    }
    __device__ void store_byte(uint32_t idx, uint32_t v) {
        if (idx < cap) buf[idx] = (uint8_t)v;
        else overflow = 1;
    }
    // Append the n low bits of v, most significant first (1 <= n <= 32).
    __device__ void put_bits(uint32_t v, uint32_t n) {
        acc |= (uint64_t)v << (64u - nacc - n);
        nacc += n;
        if (nacc >= 32u) {
            #pragma unroll
            for (uint32_t i = 0; i < 4u; i++) store_byte(byte + i, (uint32_t)(acc >> (56u - 8u * i)) & 0xFFu);
            byte += 4u;
            acc <<= 32;
            nacc -= 32u;
        }
    }
    __device__ void put(uint32_t bit) { put_bits(bit, 1u); }
    // n copies of `bit` (any n).
    __device__ void put_run(uint32_t bit, uint32_t n) {
        while (n >= 32u) { put_bits(bit ? 0xFFFFFFFFu : 0u, 32u); n -= 32u; }
        if (n) put_bits(bit ? (1u << n) - 1u : 0u, n);
    }
    // Stores the remaining bytes (the last one partial); returns the new bit offset.
    __device__ uint32_t close() {
        while (nacc >= 8u) {
            store_byte(byte, (uint32_t)(acc >> 56));
            acc <<= 8;
            nacc -= 8u;
            byte++;
        }
        if (nacc) store_byte(byte, (uint32_t)(acc >> 56));
        return byte * 8u + nacc;
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
    // The next n bits as an integer, first bit most significant (n <= 31).
    __device__ uint32_t get_bits(uint32_t n) {
        uint32_t v = 0;
        for (uint32_t i = 0; i < n; i++) v = (v << 1) | get();
        return v;
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
    // The next n bits as an integer, first bit most significant (n <= 31):
    // one shift out of the window when it holds them, else bit by bit.
    __device__ uint32_t get_bits(uint32_t n) {
        if (n == 0u) return 0u;
        const uint32_t off = pos - base;
        if (off + n <= 64u) {
            pos += n;
            return (uint32_t)((w << off) >> (64u - n));
        }
        uint32_t v = 0;
        for (uint32_t i = 0; i < n; i++) v = (v << 1) | get();
        return v;
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

// Renormalisation in closed form, the same bits and state as the spec's loop
// (cpu_reference.py:91-147, one E1/E2/E3 step per iteration):
//  * E1/E2 shift out the leading bits low and high share, n1 = clz(low ^ high)
//    of them (the narrowed interval is >= 64 wide, so n1 <= 26). The first
//    one is followed by the pending (E3) complements, the others by none.
//  * Then low = 01..., high = 10... and E3 repeats while low holds 1 and high
//    0 in the next bit down: k = the run of such positions from bit 30. Each
//    E3 step maps x to 2 (x - 2^30) = (x << 1) ^ 2^31, so k steps give
//    (x << k) ^ 2^31 (high also takes k one bits at the bottom). After an E3
//    step low < 2^31 <= high again, so no E1/E2 step can follow.
__device__ __forceinline__ uint32_t kr_rc_e3_run(uint32_t low, uint32_t high) {
    const uint32_t k = __clz(((~low) | high) << 1);
    return k > 30u ? 30u : k;
}

__device__ __forceinline__ void kr_rc_encode(uint32_t& low, uint32_t& high, uint32_t& pending,
                                             uint32_t c_lo, uint32_t c_hi, int prec,
                                             kr_bit_sink& sink) {
    kr_rc_narrow(low, high, c_lo, c_hi, prec);
    const uint32_t n1 = __clz(low ^ high);
    if (n1) {
        const uint32_t b0 = low >> 31;
        sink.put_bits(b0, 1u);
        sink.put_run(b0 ^ 1u, pending);
        pending = 0;
        if (n1 > 1u) sink.put_bits((low >> (32u - n1)) & ((1u << (n1 - 1u)) - 1u), n1 - 1u);
        low <<= n1;
        high = (high << n1) | ((1u << n1) - 1u);
    }
    const uint32_t k = kr_rc_e3_run(low, high);
    if (k) {
        pending += k;
        low = (low << k) ^ KR_RC_HALF;
        high = ((high << k) ^ KR_RC_HALF) | ((1u << k) - 1u);
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
    // the closed-form renormalisation of kr_rc_encode; value moves with low
    // and takes the stream's next bits at the bottom (cpu_reference.py:214-234)
    kr_rc_narrow(low, high, c_lo, c_hi, prec);
    const uint32_t n1 = __clz(low ^ high);
    if (n1) {
        low <<= n1;
        high = (high << n1) | ((1u << n1) - 1u);
        value = (value << n1) | src.get_bits(n1);
    }
    const uint32_t k = kr_rc_e3_run(low, high);
    if (k) {
        low = (low << k) ^ KR_RC_HALF;
        high = ((high << k) ^ KR_RC_HALF) | ((1u << k) - 1u);
        value = ((value << k) ^ KR_RC_HALF) | src.get_bits(k);
    }
}
