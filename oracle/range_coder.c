/*
 * Oracle (TEST INFRASTRUCTURE ONLY): the reference's 32-bit range coder in C.
 *
 * Restates krunch_ac/cpu_reference.py:91-234 (encode, RangeDecoder) with
 * 64-bit intermediates, as krunch_ac/cuda/encode_kernel.cu:108-137 and
 * decode_kernel.cu:50-110 do. Used as the CPU baseline's coder and pinned in
 * tests against oracle/range_coder.py (which is itself pinned against the
 * reference's golden bitstreams).
 *
 * Built by oracle/Makefile into oracle/lib/liboracle_rc.so. Nothing in the
 * product links it.
 */
#include <stdint.h>
#include <stddef.h>

#define ORC_FULL 0xFFFFFFFFu
#define ORC_HALF 0x80000000u
#define ORC_QUARTER 0x40000000u
#define ORC_3QUARTER 0xC0000000u

typedef struct {
    uint8_t *out;
    size_t cap;
    size_t nbytes;
    uint32_t cur;
    int n;
    int overflow;
} orc_sink;

static void sink_put(orc_sink *s, uint32_t bit, uint64_t count) {
    while (count--) {
        s->cur = (s->cur << 1) | bit;
        if (++s->n == 8) {
            if (s->nbytes < s->cap) s->out[s->nbytes] = (uint8_t)s->cur;
            else s->overflow = 1;
            s->nbytes++;
            s->cur = 0;
            s->n = 0;
        }
    }
}

/* Encode n intervals [lo[i], hi[i]) of total 2^log2_total. Returns the number
 * of bytes of the bitstream (which may exceed cap: then the output was
 * truncated and the caller must retry with a larger buffer). */
size_t orc_encode_intervals(const uint32_t *lo, const uint32_t *hi, size_t n,
                            int log2_total, uint8_t *out, size_t cap) {
    orc_sink s = {out, cap, 0, 0, 0, 0};
    uint32_t low = 0, high = ORC_FULL;
    uint64_t pending = 0;
    for (size_t i = 0; i < n; i++) {
        uint64_t span = (uint64_t)(high - low) + 1u;
        uint32_t nl = low + (uint32_t)((span * lo[i]) >> log2_total);
        uint32_t nh = low + (uint32_t)((span * hi[i]) >> log2_total) - 1u;
        low = nl;
        high = nh;
        for (;;) {
            if (high < ORC_HALF) {
                sink_put(&s, 0, 1);
                sink_put(&s, 1, pending);
                pending = 0;
                low <<= 1;
                high = (high << 1) | 1u;
            } else if (low >= ORC_HALF) {
                sink_put(&s, 1, 1);
                sink_put(&s, 0, pending);
                pending = 0;
                low = (low - ORC_HALF) << 1;
                high = ((high - ORC_HALF) << 1) | 1u;
            } else if (low >= ORC_QUARTER && high < ORC_3QUARTER) {
                pending++;
                low = (low - ORC_QUARTER) << 1;
                high = ((high - ORC_QUARTER) << 1) | 1u;
            } else {
                break;
            }
        }
    }
    uint32_t bit = (low < ORC_QUARTER) ? 0u : 1u;
    sink_put(&s, bit, 1);
    sink_put(&s, 1u - bit, pending + 1);
    if (s.n) {
        if (s.nbytes < s.cap) s.out[s.nbytes] = (uint8_t)(s.cur << (8 - s.n));
        s.nbytes++;
    }
    return s.nbytes;
}

typedef struct {
    const uint8_t *data;
    uint64_t len;
    uint64_t bitpos;
    uint32_t low, high, value;
} orc_decoder;

static uint32_t dec_bit(orc_decoder *d) {
    uint64_t byte = d->bitpos >> 3;
    uint32_t b = byte < d->len ? d->data[byte] : 0u;
    uint32_t bit = (b >> (7 - (d->bitpos & 7))) & 1u;
    d->bitpos++;
    return bit;
}

void orc_decoder_init(orc_decoder *d, const uint8_t *data, uint64_t len) {
    d->data = data;
    d->len = len;
    d->bitpos = 0;
    d->low = 0;
    d->high = ORC_FULL;
    d->value = 0;
    for (int i = 0; i < 32; i++) d->value = (d->value << 1) | dec_bit(d);
}

uint32_t orc_decoder_target(const orc_decoder *d, int log2_total) {
    uint64_t span = (uint64_t)(d->high - d->low) + 1u;
    uint64_t off = (uint64_t)(d->value - d->low) + 1u;
    return (uint32_t)(((off << log2_total) - 1u) / span);
}

void orc_decoder_consume(orc_decoder *d, uint32_t c_lo, uint32_t c_hi, int log2_total) {
    uint64_t span = (uint64_t)(d->high - d->low) + 1u;
    uint32_t nl = d->low + (uint32_t)((span * c_lo) >> log2_total);
    uint32_t nh = d->low + (uint32_t)((span * c_hi) >> log2_total) - 1u;
    d->low = nl;
    d->high = nh;
    for (;;) {
        uint32_t shift;
        if (d->high < ORC_HALF) shift = 0;
        else if (d->low >= ORC_HALF) shift = ORC_HALF;
        else if (d->low >= ORC_QUARTER && d->high < ORC_3QUARTER) shift = ORC_QUARTER;
        else break;
        d->low = (d->low - shift) << 1;
        d->high = ((d->high - shift) << 1) | 1u;
        d->value = ((d->value - shift) << 1) | dec_bit(d);
    }
}

/* Size of orc_decoder, so callers (ctypes) can allocate it opaquely. */
size_t orc_decoder_size(void) { return sizeof(orc_decoder); }

/* Decode n symbols against full CDF rows (n, V+1) uint32 (binary search as in
 * cpu_reference.py:225-234). */
void orc_decode_rows(orc_decoder *d, const uint32_t *cdf, size_t n, uint32_t V,
                     int log2_total, int32_t *syms) {
    for (size_t i = 0; i < n; i++) {
        const uint32_t *row = cdf + i * (size_t)(V + 1);
        uint32_t t = orc_decoder_target(d, log2_total);
        uint32_t lo = 0, hi = V;
        while (lo < hi) {
            uint32_t mid = (lo + hi) >> 1;
            if (row[mid + 1] <= t) lo = mid + 1;
            else hi = mid;
        }
        syms[i] = (int32_t)lo;
        orc_decoder_consume(d, row[lo], row[lo + 1], log2_total);
    }
}
