// selftest.hip - pulsar_moe_selftest / pulsar_router_selftest, the
// reference library's self-checks (pulsar_kernels.cu:6421-6460, 1271-1285):
// small device runs of the entry points compared with host mirrors written
// here from the formats' definitions. They allocate and synchronise (they
// are not on the hot path); each prints one line per case and returns 1
// when every case passes.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <vector>

#include "pk_common.h"
#include "../../include/pulsar_iq2xxs_grid.h"

namespace {

struct Rng {  // xorshift64*
    uint64_t s;
    explicit Rng(uint64_t seed) : s(seed * 0x9E3779B97F4A7C15ull + 1) {}
    uint32_t u32() {
        s ^= s >> 12;
        s ^= s << 25;
        s ^= s >> 27;
        return (uint32_t)((s * 0x2545F4914F6CDD1Dull) >> 32);
    }
    double uni() { return (u32() + 0.5) / 4294967296.0; }
    double normal() { return sqrt(-2.0 * log(uni())) * cos(6.283185307179586 * uni()); }
};

double h2d(uint16_t h) {
    const uint32_t e = (h >> 10) & 31u, m = h & 1023u;
    const double v = e == 0 ? ldexp((double)m, -24) : ldexp(1024.0 + m, (int)e - 25);
    return (h & 0x8000u) ? -v : v;
}
// f16 bits of a positive normal value (round to nearest)
uint16_t d2h(double v) {
    int e;
    const double f = frexp(v, &e);  // v = f 2^e, f in [0.5, 1)
    uint32_t m = (uint32_t)lrint(f * 2048.0);  // 11 significant bits
    if (m == 2048u) { m = 1024u; e++; }
    return (uint16_t)(((uint32_t)(e + 14) << 10) | (m & 1023u));
}

uint32_t rd32(const uint8_t *p) { uint32_t v; memcpy(&v, p, 4); return v; }
uint16_t rd16(const uint8_t *p) { uint16_t v; memcpy(&v, p, 2); return v; }

uint32_t block_bytes(uint32_t q) {
    switch (q) {
    case PULSAR_QUANT_Q2_K: return 84;
    case PULSAR_QUANT_IQ2_XXS: return 66;
    case PULSAR_QUANT_Q4_K: return 144;
    case PULSAR_QUANT_Q6_K: return 210;
    default: return 17;  // MXFP4, per 32 values
    }
}
uint64_t row_bytes_of(uint32_t q, uint32_t n) {
    return q == PULSAR_QUANT_MXFP4 ? (uint64_t)(n / 32u) * 17u : (uint64_t)(n / 256u) * block_bytes(q);
}

// Random blocks with scales in the formats' usual ranges.
void fill_row(uint32_t q, uint8_t *row, uint32_t n, Rng &r) {
    const uint64_t rb = row_bytes_of(q, n);
    for (uint64_t i = 0; i < rb; i++) row[i] = (uint8_t)r.u32();
    const uint32_t bb = block_bytes(q), nblk = (uint32_t)(rb / bb);
    for (uint32_t b = 0; b < nblk; b++) {
        uint8_t *blk = row + (uint64_t)b * bb;
        const uint16_t d = d2h(1e-3 + 9e-3 * r.uni()), dm = d2h(1e-3 + 9e-3 * r.uni());
        switch (q) {
        case PULSAR_QUANT_Q4_K: memcpy(blk, &d, 2); memcpy(blk + 2, &dm, 2); break;
        case PULSAR_QUANT_Q2_K: memcpy(blk + 80, &d, 2); memcpy(blk + 82, &dm, 2); break;
        case PULSAR_QUANT_Q6_K:
            for (int s = 0; s < 16; s++) blk[192 + s] = (uint8_t)(int8_t)((int)(r.u32() % 64u) - 32);
            memcpy(blk + 208, &d, 2);
            break;
        case PULSAR_QUANT_IQ2_XXS: memcpy(blk, &d, 2); break;
        default: blk[0] = (uint8_t)(118u + r.u32() % 9u); break;  // MXFP4 exponent
        }
    }
}

// 6-bit scale/min pair j of a Q4_K block (pulsar_kernels.cu:1349-1359)
void k4_scale_min(uint32_t j, const uint8_t *s, int *sc, int *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

// Dequantized row (double), from each format's block definition.
void dequant(uint32_t q, const uint8_t *row, uint32_t n, double *v) {
    static const uint16_t codes[256] = {PULSAR_IQ2XXS_GRID_CODES};
    static const double e2m1[8] = {0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0};
    if (q == PULSAR_QUANT_MXFP4) {
        for (uint32_t b = 0; b < n / 32u; b++) {
            const uint8_t *p = row + 17ull * b;
            const double sc = p[0] < 2 ? 0.0 : ldexp(1.0, (int)p[0] - 127);
            for (uint32_t i = 0; i < 16; i++) {
                const uint32_t lo = p[1 + i] & 15u, hi = p[1 + i] >> 4;
                v[32 * b + i] = (lo & 8 ? -1.0 : 1.0) * e2m1[lo & 7] * sc;
                v[32 * b + 16 + i] = (hi & 8 ? -1.0 : 1.0) * e2m1[hi & 7] * sc;
            }
        }
        return;
    }
    for (uint32_t b = 0; b < n / 256u; b++) {
        const uint8_t *blk = row + (uint64_t)b * block_bytes(q);
        double *o = v + 256ull * b;
        if (q == PULSAR_QUANT_Q4_K) {
            const double d = h2d(rd16(blk)), dm = h2d(rd16(blk + 2));
            for (uint32_t s = 0; s < 8; s++) {
                int sc, m;
                k4_scale_min(s, blk + 4, &sc, &m);
                for (uint32_t i = 0; i < 32; i++) {
                    const uint8_t byte = blk[16 + 32 * (s / 2) + i];
                    o[32 * s + i] = d * sc * ((s & 1) ? (byte >> 4) : (byte & 15)) - dm * m;
                }
            }
        } else if (q == PULSAR_QUANT_Q2_K) {
            const double d = h2d(rd16(blk + 80)), dm = h2d(rd16(blk + 82));
            for (uint32_t c = 0; c < 16; c++)
                for (uint32_t i = 0; i < 16; i++) {
                    const int qv = (blk[16 + 32 * (c / 8) + 16 * (c % 2) + i] >> (2 * ((c % 8) / 2))) & 3;
                    o[16 * c + i] = d * (blk[c] & 15) * qv - dm * (blk[c] >> 4);
                }
        } else if (q == PULSAR_QUANT_Q6_K) {
            const double d = h2d(rd16(blk + 208));
            for (uint32_t h = 0; h < 2; h++)
                for (uint32_t qq = 0; qq < 4; qq++)
                    for (uint32_t i = 0; i < 32; i++) {
                        const uint8_t lb = blk[64 * h + 32 * (qq & 1) + i];
                        const int lo = (qq >> 1) ? (lb >> 4) : (lb & 15);
                        const int hi = (blk[128 + 32 * h + i] >> (2 * qq)) & 3;
                        const uint32_t vi = 32 * qq + i;
                        o[128 * h + vi] = d * (int8_t)blk[192 + 8 * h + vi / 16] * ((lo | (hi << 4)) - 32);
                    }
        } else {  // IQ2_XXS
            const double d = h2d(rd16(blk));
            for (uint32_t g = 0; g < 8; g++) {
                const uint32_t a0 = rd32(blk + 2 + 8 * g), a1 = rd32(blk + 6 + 8 * g);
                const double db = 0.125 * d * (2.0 * (a1 >> 28) + 1.0);
                for (uint32_t k = 0; k < 4; k++) {
                    uint32_t s7 = (a1 >> (7 * k)) & 127u, par = 0;
                    for (uint32_t t = s7; t; t >>= 1) par ^= t & 1u;
                    const uint32_t sm = s7 | (par << 7);
                    uint32_t code = codes[(a0 >> (8 * k)) & 255u];
                    for (uint32_t i = 0; i < 8; i++) {
                        static const double mag[3] = {8.0, 25.0, 43.0};
                        const double m = mag[code % 3];
                        code /= 3;
                        o[32 * g + 8 * k + i] = ((sm >> i) & 1u) ? -db * m : db * m;
                    }
                }
            }
        }
    }
}

// q8_K rows of the CPU lane (crates/quant/src/cpu_dot.rs:26-50)
void quantize_rows(const float *x, uint32_t n, uint32_t rows, uint8_t *out) {
    const uint32_t nb = (n + 255u) / 256u;
    for (uint32_t r = 0; r < rows; r++)
        for (uint32_t b = 0; b < nb; b++) {
            uint8_t *o = out + ((uint64_t)r * nb + b) * 292u;
            float v[256], am = 0.0f;
            for (uint32_t i = 0; i < 256; i++) {
                v[i] = b * 256 + i < n ? x[(uint64_t)r * n + b * 256 + i] : 0.0f;
                am = fmaxf(am, fabsf(v[i]));
            }
            float d = 0.0f;
            int8_t qs[256] = {0};
            if (am != 0.0f) {
                d = am / 127.0f;
                const float inv = 127.0f / am;
                for (uint32_t i = 0; i < 256; i++) {
                    float qf = roundf(v[i] * inv);
                    qf = qf != qf ? 0.0f : fminf(fmaxf(qf, -127.0f), 127.0f);
                    qs[i] = (int8_t)qf;
                }
            }
            memcpy(o, &d, 4);
            memcpy(o + 4, qs, 256);
            for (uint32_t g = 0; g < 16; g++) {
                int16_t s = 0;
                for (uint32_t i = 0; i < 16; i++) s = (int16_t)(s + qs[16 * g + i]);
                memcpy(o + 260 + 2 * g, &s, 2);
            }
        }
}

void deq8(const uint8_t *xq, uint32_t n, double *v) {  // one q8_K row
    for (uint32_t b = 0; b < (n + 255u) / 256u; b++) {
        float d;
        memcpy(&d, xq + 292ull * b, 4);
        for (uint32_t i = 0; i < 256 && b * 256 + i < n; i++) v[b * 256 + i] = (double)d * (int8_t)xq[292ull * b + 4 + i];
    }
}

double glu_h(double g, double u, uint32_t op) {
    if (op == PULSAR_ACT_SWIGLU_OAI) {
        g = fmin(g, 7.0);
        u = fmin(fmax(u, -7.0), 7.0);
        return g / (1.0 + exp(-1.702 * g)) * (u + 1.0);
    }
    return g / (1.0 + exp(-g)) * u;
}

struct Dev {  // device allocations of one case, freed together
    std::vector<void *> p;
    bool ok = true;
    void *alloc(size_t n) {
        void *q = nullptr;
        if (hipMalloc(&q, n ? n : 1) != hipSuccess) { ok = false; return nullptr; }
        p.push_back(q);
        return q;
    }
    void *up(const void *h, size_t n) {
        void *q = alloc(n);
        if (q && hipMemcpy(q, h, n, hipMemcpyHostToDevice) != hipSuccess) ok = false;
        return q;
    }
    void down(void *h, const void *d, size_t n) {
        if (hipMemcpy(h, d, n, hipMemcpyDeviceToHost) != hipSuccess) ok = false;
    }
    ~Dev() { for (void *q : p) (void)hipFree(q); }
};

// max over outputs of |got - want| / (bound + tiny)
double ratio(double got, double want, double scale) { return fabs(got - want) / (1e-4 * scale + 1e-12); }

int moe_case(uint32_t q, const char *name) {
    const bool mx = q == PULSAR_QUANT_MXFP4;
    const uint32_t in = mx ? 576u : 512u, mid = mx ? 320u : 256u, E = 4, n_used = 3, n_tok = 2;
    const uint32_t act = mx ? PULSAR_ACT_SWIGLU_OAI : PULSAR_ACT_SILU;
    const uint64_t grb = row_bytes_of(q, in), drb = row_bytes_of(q, mid);
    Rng r(1000 + q);
    std::vector<uint8_t> gate(E * mid * grb), upw(E * mid * grb), dn(E * in * drb);
    for (uint32_t i = 0; i < E * mid; i++) {
        fill_row(q, &gate[i * grb], in, r);
        fill_row(q, &upw[i * grb], in, r);
    }
    for (uint32_t i = 0; i < E * in; i++) fill_row(q, &dn[i * drb], mid, r);
    std::vector<float> gb(E * mid), ub(E * mid), db(E * in), x(n_tok * in), w(n_tok * n_used);
    for (auto &v : gb) v = (float)(0.02 * r.normal());
    for (auto &v : ub) v = (float)(0.02 * r.normal());
    for (auto &v : db) v = (float)(0.02 * r.normal());
    for (auto &v : x) v = (float)r.normal();
    for (auto &v : w) v = (float)(0.1 + 0.9 * r.uni());
    const int sel[n_tok * n_used] = {2, 0, -1, 1, 3, 2};  // -1: an unrouted slot
    const uint32_t nbi = (in + 255u) / 256u, nbm = (mid + 255u) / 256u;

    Dev d;
    uint8_t *dg = (uint8_t *)d.up(gate.data(), gate.size()), *du = (uint8_t *)d.up(upw.data(), upw.size());
    uint8_t *dd = (uint8_t *)d.up(dn.data(), dn.size());
    float *dgb = (float *)d.up(gb.data(), gb.size() * 4), *dub = (float *)d.up(ub.data(), ub.size() * 4);
    float *ddb = (float *)d.up(db.data(), db.size() * 4);
    float *dx = (float *)d.up(x.data(), x.size() * 4), *dw = (float *)d.up(w.data(), w.size() * 4);
    if (!d.ok) return 0;
    std::vector<pulsar_expert_ptrs> hp(n_tok * n_used);
    for (uint32_t i = 0; i < n_tok * n_used; i++) {
        const int e = sel[i];
        hp[i] = e < 0 ? pulsar_expert_ptrs{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr}
                      : pulsar_expert_ptrs{dg + (uint64_t)e * mid * grb, du + (uint64_t)e * mid * grb,
                                           dd + (uint64_t)e * in * drb, mx ? dgb + e * mid : nullptr,
                                           mx ? dub + e * mid : nullptr, mx ? ddb + e * in : nullptr};
    }
    void *dptrs = d.up(hp.data(), hp.size() * sizeof(pulsar_expert_ptrs));
    uint8_t *dxq = (uint8_t *)d.alloc((size_t)n_tok * nbi * 292);
    float *dmid = (float *)d.alloc((size_t)n_tok * n_used * mid * 4);
    uint8_t *dmq = (uint8_t *)d.alloc((size_t)n_tok * n_used * nbm * 292);
    float *dout = (float *)d.alloc((size_t)n_tok * in * 4);
    if (!d.ok) return 0;
    int ok = pulsar_quantize_q8_K(dxq, dx, in, n_tok) &&
             pulsar_moe_pair_swiglu(dmid, dptrs, dw, dxq, in, mid, n_used, n_tok, grb, q, act) &&
             pulsar_quantize_q8_K(dmq, dmid, mid, n_tok * n_used) &&
             pulsar_moe_down(dout, dptrs, dmq, mid, in, n_used, n_tok, drb, q) &&
             (!mx || pulsar_moe_down_bias(dout, dptrs, dw, in, n_used, n_tok));
    if (!ok || hipDeviceSynchronize() != hipSuccess) return 0;
    std::vector<uint8_t> xq(n_tok * nbi * 292), hxq(n_tok * nbi * 292), mq(n_tok * n_used * nbm * 292);
    std::vector<float> gmid(n_tok * n_used * mid), gout(n_tok * in);
    d.down(xq.data(), dxq, xq.size());
    d.down(mq.data(), dmq, mq.size());
    d.down(gmid.data(), dmid, gmid.size() * 4);
    d.down(gout.data(), dout, gout.size() * 4);
    if (!d.ok) return 0;
    quantize_rows(x.data(), in, n_tok, hxq.data());
    const bool q8_ok = memcmp(xq.data(), hxq.data(), xq.size()) == 0;
    // host mirror: pair on the device's q8_K x, down on the device's mid q8_K
    double worst = 0.0;
    std::vector<double> row(in > mid ? in : mid), xv(in), mv(mid);
    for (uint32_t t = 0; t < n_tok; t++) {
        deq8(&xq[(uint64_t)t * nbi * 292], in, xv.data());
        std::vector<double> out(in, 0.0), oscale(in, 0.0);
        for (uint32_t s = 0; s < n_used; s++) {
            const uint32_t so = t * n_used + s;
            const int e = sel[so];
            for (uint32_t rr = 0; rr < mid; rr++) {
                double want = 0.0, scale = 0.0;
                if (e >= 0) {
                    double g = 0, u = 0, ag = 0, au = 0;
                    dequant(q, &gate[((uint64_t)e * mid + rr) * grb], in, row.data());
                    for (uint32_t i = 0; i < in; i++) { g += row[i] * xv[i]; ag += fabs(row[i] * xv[i]); }
                    dequant(q, &upw[((uint64_t)e * mid + rr) * grb], in, row.data());
                    for (uint32_t i = 0; i < in; i++) { u += row[i] * xv[i]; au += fabs(row[i] * xv[i]); }
                    if (mx) { g += gb[e * mid + rr]; u += ub[e * mid + rr]; }
                    want = glu_h(g, u, act) * w[so];
                    scale = w[so] * (2.0 * (fabs(u) + 1.0) * ag + (fabs(g) + 1.0) * au) + fabs(want);
                }
                const double rt = ratio(gmid[(uint64_t)so * mid + rr], want, scale);
                worst = rt > worst ? rt : worst;
            }
            if (e < 0) continue;
            deq8(&mq[(uint64_t)so * nbm * 292], mid, mv.data());
            for (uint32_t rr = 0; rr < in; rr++) {
                dequant(q, &dn[((uint64_t)e * in + rr) * drb], mid, row.data());
                for (uint32_t i = 0; i < mid; i++) { out[rr] += row[i] * mv[i]; oscale[rr] += fabs(row[i] * mv[i]); }
                if (mx) out[rr] += (double)w[so] * db[e * in + rr];
            }
        }
        for (uint32_t rr = 0; rr < in; rr++) {
            const double rt = ratio(gout[(uint64_t)t * in + rr], out[rr], oscale[rr] + fabs(out[rr]));
            worst = rt > worst ? rt : worst;
        }
    }
    const bool pass = q8_ok && worst <= 1.0;
    fprintf(stderr, "pulsar-kernels: moe selftest %s: %s (q8_K %s, worst error / 1e-4 bound %.3g)\n", name,
            pass ? "PASS" : "FAIL", q8_ok ? "bit-exact" : "MISMATCH", worst);
    return pass ? 1 : 0;
}

int router_case(uint32_t n_expert, uint32_t k, uint32_t mode, uint32_t n_sh, uint32_t n_tok) {
    Rng r(7 + n_expert * 31u + k * 7u + mode);
    const uint32_t n_logit = n_expert + (mode == 2u ? n_sh : 0u), n_slot = k + (mode == 2u ? n_sh : 0u);
    std::vector<float> lg(n_tok * n_logit), bias(n_expert);
    for (auto &v : lg) v = (float)(3.0 * r.normal());
    for (uint32_t i = 0; i < n_tok * n_logit; i += 5) lg[i] = lg[i / 5 % n_logit];  // ties
    for (auto &v : bias) v = mode == 1u ? 0.0f : (float)(0.5 * r.normal());
    Dev d;
    float *dl = (float *)d.up(lg.data(), lg.size() * 4), *db = (float *)d.up(bias.data(), bias.size() * 4);
    int32_t *dsel = (int32_t *)d.alloc((size_t)n_tok * n_slot * 4);
    float *dw = (float *)d.alloc((size_t)n_tok * n_slot * 4);
    if (!d.ok || !pulsar_router_select(dsel, dw, dl, db, n_expert, k, 1.5f, n_tok, mode, n_sh) ||
        hipDeviceSynchronize() != hipSuccess)
        return 0;
    std::vector<int32_t> sel(n_tok * n_slot);
    std::vector<float> w(n_tok * n_slot);
    d.down(sel.data(), dsel, sel.size() * 4);
    d.down(w.data(), dw, w.size() * 4);
    if (!d.ok) return 0;
    bool pass = true;
    double werr = 0.0;
    for (uint32_t t = 0; t < n_tok; t++) {
        const float *l = &lg[(uint64_t)t * n_logit];
        std::vector<float> prob(n_expert), score(n_expert);
        for (uint32_t e = 0; e < n_expert; e++) {
            // the kernel's sigmoid form (pulsar_kernels.cu:913-921)
            const float xe = l[e];
            const float sg = xe >= 0.0f ? 1.0f / (1.0f + expf(-xe)) : expf(xe) / (1.0f + expf(xe));
            const float p = mode == 1u ? xe : sg;
            prob[e] = mode == 2u ? l[e] : p;
            score[e] = p + bias[e];
        }
        std::vector<int32_t> ws(n_slot);
        std::vector<double> wv(n_slot);
        for (uint32_t kk = 0; kk < k; kk++) {  // higher score, then lower index; winners go to -inf
            int32_t best = -1;
            for (uint32_t e = 0; e < n_expert; e++)
                if (best < 0 || score[e] > score[best]) best = (int32_t)e;
            ws[kk] = best;
            wv[kk] = prob[best];
            score[best] = -INFINITY;
        }
        for (uint32_t s = 0; s < (mode == 2u ? n_sh : 0u); s++) {
            ws[k + s] = (int32_t)(n_expert + s);
            wv[k + s] = l[n_expert + s];
        }
        double sum = 0.0;
        if (mode == 0u) {
            for (uint32_t kk = 0; kk < k; kk++) sum += wv[kk];
            sum = fmax(sum, 6.103515625e-5);
            for (uint32_t kk = 0; kk < k; kk++) wv[kk] = wv[kk] / sum * 1.5;
        } else {
            double m = -INFINITY;
            for (uint32_t p = 0; p < n_slot; p++) {
                if (mode == 2u) wv[p] = wv[p] < 0.0 ? wv[p] - log1p(exp(wv[p])) : -log1p(exp(-wv[p]));
                m = fmax(m, wv[p]);
            }
            for (uint32_t p = 0; p < n_slot; p++) { wv[p] = exp(wv[p] - m); sum += wv[p]; }
            for (uint32_t p = 0; p < n_slot; p++) wv[p] = wv[p] / sum * 1.5;
        }
        for (uint32_t p = 0; p < n_slot; p++) {
            if (sel[t * n_slot + p] != ws[p]) pass = false;
            werr = fmax(werr, fabs(w[t * n_slot + p] - wv[p]));
        }
    }
    pass = pass && werr <= 1e-5;
    fprintf(stderr, "pulsar-kernels: router selftest n_expert %u k %u mode %u: %s (max weight error %.2g)\n",
            n_expert, k, mode, pass ? "PASS" : "FAIL", werr);
    return pass ? 1 : 0;
}

}  // namespace

extern "C" int pulsar_moe_selftest(void) {
    int ok = 1;
    ok &= moe_case(PULSAR_QUANT_Q2_K, "q2_K");
    ok &= moe_case(PULSAR_QUANT_IQ2_XXS, "iq2_xxs");
    ok &= moe_case(PULSAR_QUANT_Q4_K, "q4_K");
    ok &= moe_case(PULSAR_QUANT_Q6_K, "q6_K");
    ok &= moe_case(PULSAR_QUANT_MXFP4, "mxfp4");
    return ok;
}

extern "C" int pulsar_router_selftest(void) {
    int ok = 1;
    ok &= router_case(64, 8, 1, 0, 3);
    ok &= router_case(256, 8, 1, 0, 2);
    ok &= router_case(128, 6, 0, 0, 3);
    ok &= router_case(896, 16, 1, 0, 2);
    ok &= router_case(256, 6, 2, 2, 2);
    return ok;
}
