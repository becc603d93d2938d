// ns_host.cpp -- host-side pieces of the C ABI: error text, the seeded
// generator for synthetic configs, and the CPU layout converter.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "ns_ffn.h"
#include "ns_internal.hpp"

namespace ns {

namespace {
thread_local std::string g_error;
}

void set_error(const std::string &msg) { g_error = msg; }

// ---- generator ------------------------------------------------------------
// SplitMix64 (Steele, Lea, Flood 2014).  Each block / element index gets its own
// stream so that any range can be generated independently and in parallel.
namespace {
constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

struct Rng {
    uint64_t s;
    Rng(uint64_t seed, uint64_t index) : s(mix64(seed ^ mix64(index * kGolden + 0x632BE59BD9B4E019ull))) {}
    uint64_t next() {
        s += kGolden;
        return mix64(s);
    }
    double uniform() { return double(next() >> 11) * 0x1.0p-53; }  // [0,1)
    double normal() {                                               // Box-Muller, one draw
        const double u1 = 1.0 - uniform(), u2 = uniform();
        return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
    }
};

// IEEE binary16, round to nearest even.
uint16_t f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint16_t sign = uint16_t((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u);
    if (ax >= 0x477ff000u) return sign | 0x7c00u;
    if (ax < 0x38800000u) {
        if (ax < 0x33000000u) return sign;
        const uint32_t e = ax >> 23, mant = (ax & 0x7fffffu) | 0x800000u, shift = 126u - e;
        uint32_t r = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (r & 1u))) ++r;
        return sign | uint16_t(r);
    }
    uint32_t r = (((ax >> 23) - 112u) << 10) | ((ax >> 13) & 0x3ffu);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r;
    return sign | uint16_t(r);
}

uint16_t small_scale(Rng &r) { return f32_to_f16(float(std::fabs(r.normal()) * 1e-3)); }

void fill_bytes(Rng &r, uint8_t *dst, size_t n) {
    for (size_t i = 0; i < n; i += 8) {
        const uint64_t v = r.next();
        for (size_t j = 0; j < 8 && i + j < n; ++j) dst[i + j] = uint8_t(v >> (8 * j));
    }
}

void synth_q4k(uint64_t seed, uint64_t block, uint8_t *b) {
    Rng r(seed, block);
    const uint16_t d = small_scale(r), dmin = small_scale(r);
    std::memcpy(b, &d, 2);
    std::memcpy(b + 2, &dmin, 2);
    fill_bytes(r, b + 4, 12);    // scales: 12 uniform bytes == 16 uniform 6-bit values
    fill_bytes(r, b + 16, 128);  // qs: uniform nibbles
}

void synth_q6k(uint64_t seed, uint64_t block, uint8_t *b) {
    Rng r(seed, block);
    fill_bytes(r, b, 192);  // ql[128], qh[64]
    uint8_t raw[16];
    fill_bytes(r, raw, 16);
    for (int i = 0; i < 16; ++i) b[192 + i] = uint8_t(int8_t(int(raw[i] & 63) - 32));
    const uint16_t d = small_scale(r);
    std::memcpy(b + 208, &d, 2);
}

template <class F>
void parallel_for(uint64_t n, int nthreads, F &&f) {
    if (nthreads < 1) nthreads = 1;
    const uint64_t nt = std::min<uint64_t>(uint64_t(nthreads), std::max<uint64_t>(1, n / 4096 + 1));
    if (nt <= 1) {
        f(0, n);
        return;
    }
    std::vector<std::thread> th;
    for (uint64_t i = 0; i < nt; ++i)
        th.emplace_back([&, i] { f(n * i / nt, n * (i + 1) / nt); });
    for (auto &t : th) t.join();
}

bool valid_layout(int layout) {
    return layout == ROW_MAJOR || layout == NSMFFN || layout == CDNA4;
}
}  // namespace

}  // namespace ns

using namespace ns;

extern "C" const char *ns_last_error(void) { return ns::g_error.c_str(); }
extern "C" int ns_abi_version(void) { return NS_FFN_ABI_VERSION; }

extern "C" uint64_t ns_layer_seed(uint64_t seed, uint32_t layer) {
    return seed ^ (uint64_t(layer) * 0x9E3779B97F4A7C15ull);
}

extern "C" int ns_synth_blocks(int type, uint64_t seed, uint64_t first, uint64_t count, void *out,
                               int nthreads) {
    if ((type != Q4_K && type != Q6_K) || (!out && count)) {
        set_error("ns_synth_blocks: bad type or null output");
        return NS_ERR_ARG;
    }
    const uint32_t bs = block_bytes(type);
    auto *dst = static_cast<uint8_t *>(out);
    parallel_for(count, nthreads, [&](uint64_t a, uint64_t b) {
        for (uint64_t i = a; i < b; ++i) {
            if (type == Q4_K) synth_q4k(seed, first + i, dst + i * bs);
            else synth_q6k(seed, first + i, dst + i * bs);
        }
    });
    return NS_OK;
}

extern "C" int ns_synth_normal_f32(uint64_t seed, uint64_t first, uint64_t count, float *out,
                                   int nthreads) {
    if (!out && count) {
        set_error("ns_synth_normal_f32: null output");
        return NS_ERR_ARG;
    }
    parallel_for(count, nthreads, [&](uint64_t a, uint64_t b) {
        for (uint64_t i = a; i < b; ++i) {
            Rng r(seed, first + i);
            out[i] = float(r.normal());
        }
    });
    return NS_OK;
}

extern "C" int ns_synth_normal_f16(uint64_t seed, uint64_t first, uint64_t count, uint16_t *out,
                                   int nthreads) {
    if (!out && count) {
        set_error("ns_synth_normal_f16: null output");
        return NS_ERR_ARG;
    }
    parallel_for(count, nthreads, [&](uint64_t a, uint64_t b) {
        for (uint64_t i = a; i < b; ++i) {
            Rng r(seed, first + i);
            out[i] = f32_to_f16(float(r.normal()));
        }
    });
    return NS_OK;
}

// Layout conversion: copy each block's 16-byte chunks (and the Q6_K d tail)
// from their place in one layout to their place in the other.
extern "C" int ns_retile(const void *src, void *dst, int type, uint32_t cols, uint32_t rows,
                         int from_layout, int to_layout) {
    if ((type != Q4_K && type != Q6_K) || !valid_layout(from_layout) || !valid_layout(to_layout)) {
        set_error("ns_retile: bad type or layout");
        return NS_ERR_ARG;
    }
    if (cols % kQK || ((from_layout != ROW_MAJOR || to_layout != ROW_MAJOR) && rows % kRowTile)) {
        set_error("ns_retile: cols must be a multiple of 256 and rows of 64");
        return NS_ERR_SHAPE;
    }
    if (!src || !dst) {
        set_error("ns_retile: null pointer");
        return NS_ERR_ARG;
    }
    const auto *s = static_cast<const uint8_t *>(src);
    auto *d = static_cast<uint8_t *>(dst);
    const uint64_t nb = cols / kQK;
    const uint32_t nchunk = type == Q4_K ? kQ4Chunks : kQ6Chunks;
    parallel_for(rows, int(std::max(1u, std::thread::hardware_concurrency())), [&](uint64_t a, uint64_t b) {
        for (uint64_t r = a; r < b; ++r)
            for (uint64_t kb = 0; kb < nb; ++kb) {
                for (uint32_t c = 0; c < nchunk; ++c)
                    std::memcpy(d + byte_offset(type, to_layout, r, kb, nb, 16 * c),
                                s + byte_offset(type, from_layout, r, kb, nb, 16 * c), 16);
                if (type == Q6_K)
                    std::memcpy(d + byte_offset(type, to_layout, r, kb, nb, 208),
                                s + byte_offset(type, from_layout, r, kb, nb, 208), 2);
            }
    });
    return NS_OK;
}
