// gh_oracle core: worker pool, IEEE binary16 conversion, GGUF Q4_K/Q6_K dequantization.
// TEST INFRASTRUCTURE — a CPU restatement of the reference, used only as a checker.
#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

#include "gh_oracle.h"
#include "internal.h"

// ---------------------------------------------------------------------------------------
// Persistent fork-join pool. Restates backend/cpu/parallel.rs:59-102 (for_units: contiguous
// chunks aligned to `stride`, chunk_units = ceil(units / n), slot 0 runs on the caller) and
// backend/cpu/pool.rs:121-156 (persistent workers, caller blocks until all slots finish).
// Only the chunking matters for the numerics: each unit is computed by one thread in a
// fixed order, so the result is independent of the worker count.
namespace gho {

static std::atomic<int> g_threads{0};

int threads() {
    int t = g_threads.load();
    if (t <= 0) {
        const char* env = std::getenv("GHO_THREADS");
        t = env ? std::atoi(env) : 0;
        if (t <= 0) t = (int)std::max(1u, std::thread::hardware_concurrency());
        g_threads.store(t);
    }
    return t;
}

namespace {
struct Pool {
    std::vector<std::thread> workers;
    std::mutex mu;
    std::condition_variable cv, done_cv;
    const std::function<void(size_t)>* job = nullptr;
    size_t nslots = 0;
    size_t next = 0;
    size_t finished = 0;
    uint64_t generation = 0;
    bool stop = false;

    explicit Pool(int n) {
        for (int i = 1; i < n; ++i) workers.emplace_back([this] { run(); });
    }
    ~Pool() {
        {
            std::lock_guard<std::mutex> g(mu);
            stop = true;
        }
        cv.notify_all();
        for (auto& w : workers) w.join();
    }
    void run() {
        uint64_t seen = 0;
        for (;;) {
            std::unique_lock<std::mutex> lk(mu);
            cv.wait(lk, [&] { return stop || generation != seen; });
            if (stop) return;
            seen = generation;
            while (next < nslots) {
                size_t slot = next++;
                const auto* f = job;
                lk.unlock();
                (*f)(slot);
                lk.lock();
                if (++finished == nslots) done_cv.notify_all();
            }
        }
    }
    void dispatch(size_t n, const std::function<void(size_t)>& f) {
        std::unique_lock<std::mutex> lk(mu);
        job = &f;
        nslots = n;
        next = 0;
        finished = 0;
        ++generation;
        cv.notify_all();
        // The caller participates like slot 0 of the reference pool.
        while (next < nslots) {
            size_t slot = next++;
            lk.unlock();
            f(slot);
            lk.lock();
            ++finished;
        }
        done_cv.wait(lk, [&] { return finished == nslots; });
        job = nullptr;
    }
};

Pool& pool() {
    static Pool* p = new Pool(threads());
    return *p;
}
std::mutex g_dispatch_mu;  // the reference pool serializes dispatchers (pool.rs:121-129)
}  // namespace

void for_units(size_t len, size_t stride, const std::function<void(size_t, size_t, size_t)>& f) {
    size_t units = stride ? len / stride : 0;
    size_t n = std::min<size_t>((size_t)threads(), units);
    if (n <= 1) {
        f(0, 0, len);
        return;
    }
    size_t chunk_units = (units + n - 1) / n;
    size_t chunk_elems = chunk_units * stride;
    size_t nslots = (units + chunk_units - 1) / chunk_units;
    std::function<void(size_t)> job = [&](size_t slot) {
        size_t start = slot * chunk_elems;
        size_t end = std::min(start + chunk_elems, len);
        f(slot * chunk_units, start, end);
    };
    std::lock_guard<std::mutex> g(g_dispatch_mu);
    pool().dispatch(nslots, job);
}

// ---------------------------------------------------------------------------------------
// binary16 <-> binary32, restating backend/f16.rs:11-71 bit for bit.
float f16_to_f32(uint16_t h) {
    uint32_t sign = (h >> 15) & 1;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t mant = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign << 31;
        } else {
            int32_t e = -1;
            uint32_t m = mant;
            while ((m & 0x400) == 0) {
                m <<= 1;
                e -= 1;
            }
            m &= 0x3ff;
            uint32_t exp32 = (uint32_t)(127 - 15 + 2 + e);
            bits = (sign << 31) | (exp32 << 23) | (m << 13);
        }
    } else if (exp == 0x1f) {
        bits = (sign << 31) | (0xffu << 23) | (mant << 13);
    } else {
        bits = (sign << 31) | ((exp + (127 - 15)) << 23) | (mant << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

uint16_t f32_to_f16(float f) {
    uint32_t bits;
    std::memcpy(&bits, &f, 4);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000);
    int32_t exp = (int32_t)((bits >> 23) & 0xff);
    uint32_t mant = bits & 0x7fffff;
    if (exp == 0xff) return (uint16_t)(sign | 0x7c00 | (mant != 0 ? 0x200 : 0));
    int32_t e = exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00);
    if (e <= 0) {
        if (e < -10) return sign;
        uint32_t m = mant | 0x800000;
        uint32_t shift = (uint32_t)(14 - e);
        uint16_t half = (uint16_t)(m >> shift);
        uint32_t rem = m & ((1u << shift) - 1);
        uint16_t round =
            (rem > (1u << (shift - 1)) || (rem == (1u << (shift - 1)) && (half & 1) == 1)) ? 1 : 0;
        return (uint16_t)(sign | (uint16_t)(half + round));
    }
    uint16_t half = (uint16_t)(((uint16_t)e << 10) | (uint16_t)(mant >> 13));
    uint32_t rem = mant & 0x1fff;
    uint16_t round = (rem > 0x1000 || (rem == 0x1000 && (half & 1) == 1)) ? 1 : 0;
    return (uint16_t)(sign | (uint16_t)(half + round));
}

// Slice widening: backend/cpu/f16.rs:131-168 (F16C bulk, exact, identical to the scalar).
__attribute__((target("avx2,f16c"))) void f16_slice_to_f32(const uint16_t* src, float* dst,
                                                            size_t n) {
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        __m128i raw = _mm_loadu_si128((const __m128i*)(src + i));
        _mm256_storeu_ps(dst + i, _mm256_cvtph_ps(raw));
    }
    for (; i < n; ++i) dst[i] = f16_to_f32(src[i]);
}

// Slice narrowing: backend/cpu/f16.rs:176-218 (F16C RNE bulk + scalar tail).
__attribute__((target("avx2,f16c"))) void f32_slice_to_f16(const float* src, uint16_t* dst,
                                                            size_t n) {
    size_t i = 0;
    for (; i + 8 <= n; i += 8) {
        __m256 f = _mm256_loadu_ps(src + i);
        __m128i h = _mm256_cvtps_ph(f, _MM_FROUND_TO_NEAREST_INT);
        _mm_storeu_si128((__m128i*)(dst + i), h);
    }
    for (; i < n; ++i) dst[i] = f32_to_f16(src[i]);
}

// ---------------------------------------------------------------------------------------
// Dequantization: backend/cpu/dequant.rs.

// scale_min, dequant.rs:78-89.
void scale_min(const uint8_t* sc12, uint32_t j, uint32_t* sc, uint32_t* mn) {
    if (j < 4) {
        *sc = sc12[j] & 63;
        *mn = sc12[j + 4] & 63;
    } else {
        uint32_t hi = sc12[j + 4];
        uint32_t lo = sc12[j - 4];
        *sc = (hi & 0xF) | ((lo >> 6) << 4);
        *mn = (hi >> 4) | (((uint32_t)sc12[j] >> 6) << 4);
    }
}

static inline float f16_at(const uint8_t* b) {
    return f16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
}

// dequant_row_q4_k, dequant.rs:93-123: w = (d*sc)*q - dmin*mn, mul then sub (two roundings).
static void dequant_row_q4_k(const uint8_t* bytes, size_t row, size_t in_dim, float* out) {
    size_t nsb = in_dim / 256;
    size_t base = row * nsb * 144;
    for (size_t s = 0; s < nsb; ++s) {
        const uint8_t* blk = bytes + base + s * 144;
        float d = f16_at(blk);
        float dmin = f16_at(blk + 2);
        const uint8_t* sco = blk + 4;
        const uint8_t* qso = blk + 16;
        size_t abase = s * 256;
        uint32_t is = 0, qb = 0;
        for (size_t j = 0; j < 256; j += 64) {
            uint32_t sc1, mn1, sc2, mn2;
            scale_min(sco, is, &sc1, &mn1);
            scale_min(sco, is + 1, &sc2, &mn2);
            float d1 = d * (float)sc1;
            float m1 = dmin * (float)mn1;
            float d2 = d * (float)sc2;
            float m2 = dmin * (float)mn2;
            for (size_t l = 0; l < 32; ++l) {
                uint32_t qv = qso[qb + l];
                out[abase + j + l] = d1 * (float)(qv & 0xF) - m1;
                out[abase + j + 32 + l] = d2 * (float)(qv >> 4) - m2;
            }
            qb += 32;
            is += 2;
        }
    }
}

// dequant_row_q6_k_scalar, dequant.rs:274-308: q = (ql nibble | qh 2 bits << 4) - 32,
// w = (d * scale) * q. The AVX2 variant (dequant.rs:319-410) is bit-identical to it.
static void dequant_row_q6_k(const uint8_t* bytes, size_t row, size_t in_dim, float* out) {
    size_t nsb = in_dim / 256;
    size_t base = row * nsb * 210;
    for (size_t s = 0; s < nsb; ++s) {
        const uint8_t* blk = bytes + base + s * 210;
        const uint8_t* qlo = blk;
        const uint8_t* qho = blk + 128;
        const uint8_t* sco = blk + 192;
        float d = f16_at(blk + 208);
        size_t abase = s * 256;
        for (size_t n = 0; n < 256; n += 128) {
            size_t seg = n / 128;
            const uint8_t* qlb = qlo + seg * 64;
            const uint8_t* qhb = qho + seg * 32;
            const int8_t* scb = (const int8_t*)(sco + seg * 8);
            for (size_t l = 0; l < 32; ++l) {
                size_t is = l / 16;
                uint32_t lo0 = qlb[l], lo1 = qlb[l + 32], h = qhb[l];
                int32_t q1 = (int32_t)((lo0 & 0xF) | ((h & 3) << 4)) - 32;
                int32_t q2 = (int32_t)((lo1 & 0xF) | (((h >> 2) & 3) << 4)) - 32;
                int32_t q3 = (int32_t)((lo0 >> 4) | (((h >> 4) & 3) << 4)) - 32;
                int32_t q4 = (int32_t)((lo1 >> 4) | (((h >> 6) & 3) << 4)) - 32;
                out[abase + n + l] = d * (float)scb[is] * (float)q1;
                out[abase + n + l + 32] = d * (float)scb[is + 2] * (float)q2;
                out[abase + n + l + 64] = d * (float)scb[is + 4] * (float)q3;
                out[abase + n + l + 96] = d * (float)scb[is + 6] * (float)q4;
            }
        }
    }
}

// dequant_row dispatch, dequant.rs:47-67.
int dequant_row(uint32_t format, const uint8_t* bytes, size_t row, size_t in_dim, float* out) {
    switch (format) {
        case FMT_F16: {
            const uint8_t* b = bytes + row * in_dim * 2;
            for (size_t i = 0; i < in_dim; ++i) out[i] = f16_at(b + i * 2);
            return 0;
        }
        case FMT_Q4_K:
            dequant_row_q4_k(bytes, row, in_dim, out);
            return 0;
        case FMT_Q6_K:
            dequant_row_q6_k(bytes, row, in_dim, out);
            return 0;
        default:
            return -1;
    }
}

size_t block_len(uint32_t format) {
    switch (format) {
        case FMT_F16: return 2;
        case FMT_Q4_K: return 144;
        case FMT_Q6_K: return 210;
        case FMT_F32: return 4;
        default: return 0;
    }
}

}  // namespace gho

extern "C" {
void gho_set_threads(int n) { gho::g_threads.store(n); }
int gho_threads(void) { return gho::threads(); }
float gho_f16_to_f32(uint16_t h) { return gho::f16_to_f32(h); }
uint16_t gho_f32_to_f16(float f) { return gho::f32_to_f16(f); }
void gho_f16_to_f32_slice(const uint16_t* s, float* d, size_t n) { gho::f16_slice_to_f32(s, d, n); }
void gho_f32_to_f16_slice(const float* s, uint16_t* d, size_t n) { gho::f32_slice_to_f16(s, d, n); }
void gho_scale_min(const uint8_t* sc12, uint32_t j, uint32_t* sc, uint32_t* mn) {
    gho::scale_min(sc12, j, sc, mn);
}
int gho_dequant_row(uint32_t format, const uint8_t* bytes, size_t row, size_t in_dim, float* out) {
    return gho::dequant_row(format, bytes, row, in_dim, out);
}
// validate, dequant.rs:35-41: a quantized weight must be a whole number of blocks.
int gho_validate(uint32_t format, size_t byte_len) {
    size_t bl = gho::block_len(format);
    if (bl == 0 || byte_len % bl != 0) return -1;
    return 0;
}
}
