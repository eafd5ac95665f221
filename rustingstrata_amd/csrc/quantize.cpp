// Host weight quantizers: f32 rows -> GGUF blocks (strata_quantize_rows). The reference ships none for these
// types (src/quant/mod.rs:1-2 only decodes). These are simple min/max fits, written for synthetic weights: any
// valid packing serves, since parity is checked on the bytes whatever produced them. The packings follow the
// decoders of src/quant/mod.rs (Q8_0 86, Q2_K 156-170, Q3_K 173-207, Q4_K 209-221, Q5_K 223-237, Q6_K 239-256,
// IQ4_XS 363-376).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/strata_hip.h"

namespace {

uint16_t f2h(float f) {
    _Float16 h = (_Float16)f;
    uint16_t b;
    std::memcpy(&b, &h, 2);
    return b;
}
float h2f(uint16_t b) {
    _Float16 h;
    std::memcpy(&h, &b, 2);
    return (float)h;
}
void put16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }
int clampi(int v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : v; }

void q8_0(const float* x, uint8_t* b) {
    float amax = 0;
    for (int i = 0; i < 32; i++) amax = std::max(amax, std::fabs(x[i]));
    uint16_t dh = f2h(amax / 127.0f);
    float d = h2f(dh), id = d > 0 ? 1.0f / d : 0.0f;
    put16(b, dh);
    for (int i = 0; i < 32; i++) b[2 + i] = (uint8_t)(int8_t)clampi((int)std::lrint(x[i] * id), -127, 127);
}

// 6-bit scales and mins of 8 sub-blocks into the 12-byte K-quant header (inverse of scale_min_k4).
void pack_k4(const int* sc, const int* mn, uint8_t* q) {
    for (int j = 0; j < 4; j++) {
        q[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        q[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
        q[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4));
    }
}

// Q4_K (levels 15) and Q5_K (levels 31): per 32 values x ~ d sc q - dmin m with q in 0..levels.
void qk_min(const float* x, uint8_t* b, int levels) {
    float scale[8], minv[8];
    for (int j = 0; j < 8; j++) {
        float lo = 0, hi = 0;
        for (int i = 0; i < 32; i++) { lo = std::min(lo, x[32 * j + i]); hi = std::max(hi, x[32 * j + i]); }
        scale[j] = (hi - lo) / levels;
        minv[j] = -lo;
    }
    float ms = *std::max_element(scale, scale + 8), mm = *std::max_element(minv, minv + 8);
    uint16_t dh = f2h(ms / 63.0f), mh = f2h(mm / 63.0f);
    float d = h2f(dh), dmin = h2f(mh);
    int sc[8], mn[8];
    for (int j = 0; j < 8; j++) {
        sc[j] = d > 0 ? clampi((int)std::lrint(scale[j] / d), 0, 63) : 0;
        mn[j] = dmin > 0 ? clampi((int)std::lrint(minv[j] / dmin), 0, 63) : 0;
    }
    put16(b, dh);
    put16(b + 2, mh);
    pack_k4(sc, mn, b + 4);
    uint8_t q[256];
    for (int j = 0; j < 8; j++) {
        float ds = d * sc[j], mv = dmin * mn[j];
        for (int i = 0; i < 32; i++) q[32 * j + i] = ds > 0 ? (uint8_t)clampi((int)std::lrint((x[32 * j + i] + mv) / ds), 0, levels) : 0;
    }
    if (levels == 15) {
        for (int p = 0; p < 4; p++)
            for (int l = 0; l < 32; l++) b[16 + 32 * p + l] = (uint8_t)(q[64 * p + l] | (q[64 * p + 32 + l] << 4));
    } else {
        std::memset(b + 16, 0, 32);
        for (int p = 0; p < 4; p++)
            for (int l = 0; l < 32; l++) {
                uint8_t a = q[64 * p + l], c = q[64 * p + 32 + l];
                b[48 + 32 * p + l] = (uint8_t)((a & 15) | ((c & 15) << 4));
                b[16 + l] |= (uint8_t)(((a >> 4) << (2 * p)) | ((c >> 4) << (2 * p + 1)));
            }
    }
}

// Q6_K: per 16 values x ~ d sc (q - 32), sc int8, q in 0..63.
void q6k(const float* x, uint8_t* b) {
    float scale[16];
    for (int g = 0; g < 16; g++) {
        float amax = 0, v = 0;
        for (int i = 0; i < 16; i++) if (std::fabs(x[16 * g + i]) > amax) { amax = std::fabs(x[16 * g + i]); v = x[16 * g + i]; }
        scale[g] = v / -32.0f;  // the largest magnitude maps to q - 32 = -32
    }
    float smax = 0;
    for (int g = 0; g < 16; g++) smax = std::max(smax, std::fabs(scale[g]));
    uint16_t dh = f2h(smax / 127.0f);
    float d = h2f(dh);
    int8_t sc[16];
    for (int g = 0; g < 16; g++) sc[g] = d > 0 ? (int8_t)clampi((int)std::lrint(scale[g] / d), -127, 127) : 0;
    uint8_t q[256];
    for (int i = 0; i < 256; i++) {
        float ds = d * sc[i / 16];
        q[i] = ds != 0 ? (uint8_t)(clampi((int)std::lrint(x[i] / ds), -32, 31) + 32) : 32;
    }
    std::memset(b, 0, 210);
    for (int n = 0; n < 2; n++) {
        const uint8_t* qn = q + 128 * n;
        uint8_t *ql = b + 64 * n, *qh = b + 128 + 32 * n;
        for (int l = 0; l < 32; l++) {
            ql[l] = (uint8_t)((qn[l] & 15) | ((qn[l + 64] & 15) << 4));
            ql[l + 32] = (uint8_t)((qn[l + 32] & 15) | ((qn[l + 96] & 15) << 4));
            qh[l] = (uint8_t)((qn[l] >> 4) | ((qn[l + 32] >> 4) << 2) | ((qn[l + 64] >> 4) << 4) | ((qn[l + 96] >> 4) << 6));
        }
    }
    for (int g = 0; g < 16; g++) b[192 + g] = (uint8_t)sc[g];
    put16(b + 208, dh);
}

// Q2_K: per 16 values x ~ d sc q - dmin m with q in 0..3, sc and m 4 bits.
void q2k(const float* x, uint8_t* b) {
    float scale[16], minv[16];
    for (int g = 0; g < 16; g++) {
        float lo = 0, hi = 0;
        for (int i = 0; i < 16; i++) { lo = std::min(lo, x[16 * g + i]); hi = std::max(hi, x[16 * g + i]); }
        scale[g] = (hi - lo) / 3;
        minv[g] = -lo;
    }
    float ms = *std::max_element(scale, scale + 16), mm = *std::max_element(minv, minv + 16);
    uint16_t dh = f2h(ms / 15.0f), mh = f2h(mm / 15.0f);
    float d = h2f(dh), dmin = h2f(mh);
    uint8_t q[256];
    for (int g = 0; g < 16; g++) {
        int s = d > 0 ? clampi((int)std::lrint(scale[g] / d), 0, 15) : 0;
        int m = dmin > 0 ? clampi((int)std::lrint(minv[g] / dmin), 0, 15) : 0;
        b[g] = (uint8_t)(s | (m << 4));
        float ds = d * s, mv = dmin * m;
        for (int i = 0; i < 16; i++) q[16 * g + i] = ds > 0 ? (uint8_t)clampi((int)std::lrint((x[16 * g + i] + mv) / ds), 0, 3) : 0;
    }
    std::memset(b + 16, 0, 64);
    // value i: byte 16 + 32 (i / 128) + i % 32, bits 2 ((i / 32) % 4)
    for (int i = 0; i < 256; i++) b[16 + 32 * (i / 128) + i % 32] |= (uint8_t)(q[i] << (2 * ((i / 32) % 4)));
    put16(b + 80, dh);
    put16(b + 82, mh);
}

// Q3_K: per 16 values x ~ d (sc - 32) (q - 4) with q in 0..7 (2 low bits + hmask bit), sc 6 bits.
void q3k(const float* x, uint8_t* b) {
    float scale[16];
    for (int g = 0; g < 16; g++) {
        float amax = 0, v = 0;
        for (int i = 0; i < 16; i++) if (std::fabs(x[16 * g + i]) > amax) { amax = std::fabs(x[16 * g + i]); v = x[16 * g + i]; }
        scale[g] = v / -4.0f;
    }
    float smax = 0;
    for (int g = 0; g < 16; g++) smax = std::max(smax, std::fabs(scale[g]));
    uint16_t dh = f2h(smax / 31.0f);
    float d = h2f(dh);
    int sc[16];
    for (int g = 0; g < 16; g++) sc[g] = d > 0 ? clampi((int)std::lrint(scale[g] / d), -32, 31) : 0;
    std::memset(b, 0, 110);
    for (int i = 0; i < 256; i++) {
        float ds = d * sc[i / 16];
        int q = ds != 0 ? clampi((int)std::lrint(x[i] / ds), -4, 3) + 4 : 4;
        int k = (i / 32) % 4 + 4 * (i / 128);
        b[32 + 32 * (i / 128) + i % 32] |= (uint8_t)((q & 3) << (2 * (k % 4)));
        if (q & 4) b[i % 32] |= (uint8_t)(1 << k);
    }
    // 12 scale bytes (inverse of q3k_scales): low nibbles in bytes 0..7, high 2 bits in bytes 8..11.
    for (int is = 0; is < 16; is++) {
        int v = sc[is] + 32;
        b[96 + (is & 7)] |= (uint8_t)((v & 15) << (4 * (is >> 3)));
        b[96 + 8 + (is & 3)] |= (uint8_t)(((v >> 4) & 3) << (2 * (is >> 2)));
    }
    put16(b + 108, dh);
}

// IQ4_XS: per 32 values x ~ d (ls - 32) KVALUES[nibble], ls 6 bits.
void iq4xs(const float* x, uint8_t* b) {
    static const int kv[16] = {-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113};
    float scale[8];
    for (int j = 0; j < 8; j++) {
        float amax = 0, v = 0;
        for (int i = 0; i < 32; i++) if (std::fabs(x[32 * j + i]) > amax) { amax = std::fabs(x[32 * j + i]); v = x[32 * j + i]; }
        scale[j] = v / -127.0f;
    }
    float smax = 0;
    for (int j = 0; j < 8; j++) smax = std::max(smax, std::fabs(scale[j]));
    uint16_t dh = f2h(smax / 31.0f);
    float d = h2f(dh);
    std::memset(b, 0, 136);
    put16(b, dh);
    uint16_t sh = 0;
    for (int j = 0; j < 8; j++) {
        int ls = (d > 0 ? clampi((int)std::lrint(scale[j] / d), -32, 31) : 0) + 32;
        b[4 + j / 2] |= (uint8_t)((ls & 15) << (4 * (j % 2)));
        sh |= (uint16_t)(((ls >> 4) & 3) << (2 * j));
        float dl = d * (ls - 32);
        for (int i = 0; i < 32; i++) {
            int best = 0;
            float be = INFINITY;
            for (int c = 0; c < 16; c++) {
                float e = std::fabs(dl * kv[c] - x[32 * j + i]);
                if (e < be) { be = e; best = c; }
            }
            int l = i % 16;
            b[8 + 16 * j + l] |= (uint8_t)(best << (i < 16 ? 0 : 4));
        }
    }
    put16(b + 2, sh);
}

}  // namespace

extern "C" uint64_t strata_row_bytes(int ty, uint64_t cols);
extern "C" const char* strata_last_error(void);

extern "C" int strata_quantize_rows(int ty, const float* src, uint64_t rows, uint64_t cols, uint8_t* dst) {
    uint64_t be = ty == 8 ? 32 : 256;
    uint64_t rb = strata_row_bytes(ty, cols);
    if (!rb || cols % be || !(ty == 8 || ty == 10 || ty == 11 || ty == 12 || ty == 13 || ty == 14 || ty == 23)) return -1;
    uint64_t nb = cols / be, bb = rb / nb;
    auto work = [&](uint64_t r0, uint64_t r1) {
        for (uint64_t r = r0; r < r1; r++)
            for (uint64_t k = 0; k < nb; k++) {
                const float* x = src + r * cols + k * be;
                uint8_t* b = dst + r * rb + k * bb;
                switch (ty) {
                case 8: q8_0(x, b); break;
                case 10: q2k(x, b); break;
                case 11: q3k(x, b); break;
                case 12: qk_min(x, b, 15); break;
                case 13: qk_min(x, b, 31); break;
                case 14: q6k(x, b); break;
                case 23: iq4xs(x, b); break;
                }
            }
    };
    unsigned nth = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    if (rows < 64) nth = 1;
    std::vector<std::thread> th;
    uint64_t per = (rows + nth - 1) / nth;
    for (unsigned i = 0; i < nth; i++) {
        uint64_t r0 = i * per, r1 = std::min(rows, r0 + per);
        if (r0 < r1) th.emplace_back(work, r0, r1);
    }
    for (auto& t : th) t.join();
    return 0;
}
