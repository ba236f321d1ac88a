/* Body of the oracle, included twice by attn_oracle.c with REAL = double / float.
 * TEST INFRASTRUCTURE ONLY (see attn_oracle.c). */

/* metal/clef.metal:245-300 (attn_prep). qkv [T][row] holds [nh x (q | gate)] [nkv K] [nkv V]. */
void SFX(orc_text_prep)(int T, int nh, int nkv, int hd, int n_rot, int row, double eps,
                        const float *qkv, const float *qnorm, const float *knorm,
                        const int32_t *pos3, const float *inv_freq,
                        REAL *Q, REAL *K, REAL *V, REAL *G) {
    const int half = n_rot / 2;
#pragma omp parallel for collapse(2) schedule(static)
    for (int t = 0; t < T; t++) {
        for (int head = 0; head < nh + nkv; head++) {
            const float *r = qkv + (size_t)t * row;
            const int is_q = head < nh, kh = head - nh;
            const float *src = is_q ? r + (size_t)head * 2 * hd : r + (size_t)nh * 2 * hd + (size_t)kh * hd;
            const float *w = is_q ? qnorm : knorm;
            REAL *dst = is_q ? Q + ((size_t)head * T + t) * hd : K + ((size_t)kh * T + t) * hd;
            REAL ss = 0;
            for (int d = 0; d < hd; d++) ss += (REAL)src[d] * (REAL)src[d];
            /* w == NULL: no RMSNorm (plain SDPA operands) */
            const REAL inv = w ? (REAL)1 / sqrt(ss / (REAL)hd + (REAL)eps) : (REAL)1;
            for (int d = 0; d < hd; d++) dst[d] = (REAL)src[d] * inv * (w ? (REAL)w[d] : (REAL)1);
            for (int i = 0; i < half; i++) {
                /* angle in f32 as the reference computes it: (float)pos * inv_freq[i] */
                const float ang = (float)pos3[3 * (size_t)t + i % 3] * inv_freq[i];
                const REAL c = cos((REAL)ang), s = sin((REAL)ang);
                const REAL x0 = dst[i], x1 = dst[i + half];
                dst[i] = x0 * c - x1 * s;
                dst[i + half] = x1 * c + x0 * s;
            }
            if (is_q) {
                for (int d = 0; d < hd; d++) G[(size_t)t * nh * hd + (size_t)head * hd + d] = (REAL)src[hd + d];
            } else {
                const float *vs = r + (size_t)nh * 2 * hd + (size_t)nkv * hd + (size_t)kh * hd;
                for (int d = 0; d < hd; d++) V[((size_t)kh * T + t) * hd + d] = (REAL)vs[d];
            }
        }
    }
}

/* ref/safe_attn.py:25-68 semantics over packed records. Q [nh][Tq][hd], K/V [nkv][Tk][hd],
 * record r's queries are rows cu_q[r]..cu_q[r+1], its keys rows cu_k[r]..cu_k[r+1] (cu_k NULL:
 * cu_q). With L = keys - queries, query j sees keys 0..L+j (causal) or all keys. G [Tq][nh*hd]
 * (nullable) multiplies the output by sigmoid(G) (metal/clef.metal:316-352). O [Tq][nh*hd]. */
/* rows != NULL: only those query rows are computed, O is then [n_rows][nh*hd]. */
void SFX(orc_attention)(int nh, int nkv, int hd, int Tq, int Tk, const REAL *Q, const REAL *K,
                        const REAL *V, const int32_t *cu_q, const int32_t *cu_k, int n_seq,
                        int causal, double scale, const REAL *G, REAL *O,
                        const int32_t *rows, int n_rows) {
    if (!cu_k) cu_k = cu_q;
    const int grp = nh / nkv;
#pragma omp parallel
    {
        int maxk = 1;
        for (int r = 0; r < n_seq; r++)
            if (cu_k[r + 1] - cu_k[r] > maxk) maxk = cu_k[r + 1] - cu_k[r];
        REAL *sc = (REAL *)malloc(sizeof(REAL) * (size_t)maxk);
        REAL *acc = (REAL *)malloc(sizeof(REAL) * (size_t)hd);
        const int n_out = rows ? n_rows : Tq;
#pragma omp for collapse(2) schedule(dynamic, 16)
        for (int h = 0; h < nh; h++) {
            for (int ti = 0; ti < n_out; ti++) {
                const int t = rows ? rows[ti] : ti;
                int r = 0;
                while (r < n_seq && cu_q[r + 1] <= t) r++;
                const int nq = cu_q[r + 1] - cu_q[r], nk = cu_k[r + 1] - cu_k[r];
                const int j = t - cu_q[r], L = nk - nq;
                const int last = causal ? L + j : nk - 1;
                const int kh = h / grp;
                const REAL *q = Q + ((size_t)h * Tq + t) * hd;
                const REAL *Kr = K + ((size_t)kh * Tk + cu_k[r]) * hd;
                const REAL *Vr = V + ((size_t)kh * Tk + cu_k[r]) * hd;
                REAL mx = -INFINITY;
                for (int s = 0; s <= last; s++) {
                    REAL dot = 0;
                    const REAL *k = Kr + (size_t)s * hd;
                    for (int d = 0; d < hd; d++) dot += q[d] * k[d];
                    sc[s] = dot * (REAL)scale;
                    if (sc[s] > mx) mx = sc[s];
                }
                REAL sum = 0;
                for (int d = 0; d < hd; d++) acc[d] = 0;
                for (int s = 0; s <= last; s++) {
                    const REAL p = exp(sc[s] - mx);
                    sum += p;
                    const REAL *v = Vr + (size_t)s * hd;
                    for (int d = 0; d < hd; d++) acc[d] += p * v[d];
                }
                REAL *o = O + (size_t)ti * nh * hd + (size_t)h * hd;
                /* a row with no visible key is defined as zero (ref/safe_attn.py:38-40) */
                const REAL inv = last >= 0 && sum > 0 ? (REAL)1 / sum : (REAL)0;
                for (int d = 0; d < hd; d++) {
                    REAL val = acc[d] * inv;
                    if (G) val *= (REAL)1 / ((REAL)1 + exp(-G[(size_t)t * nh * hd + (size_t)h * hd + d]));
                    o[d] = val;
                }
            }
        }
        free(sc);
        free(acc);
    }
}

/* metal/clef.metal:1616-1656 (vis_qkv_rope). qkv [P][3E], E = heads*hd, bias [3E] or NULL,
 * pos2 [P][2] = (grid row, grid column), inv_freq [hd/4]. Q/K/V [heads][P][hd]. */
void SFX(orc_vis_prep)(int P, int heads, int hd, const float *qkv, const float *bias,
                       const int32_t *pos2, const float *inv_freq, REAL *Q, REAL *K, REAL *V) {
    const int E = heads * hd, rot = hd / 2, quarter = hd / 4;
#pragma omp parallel for collapse(2) schedule(static)
    for (int p = 0; p < P; p++) {
        for (int h = 0; h < heads; h++) {
            const float *row = qkv + (size_t)p * 3 * E;
            const size_t o = ((size_t)h * P + p) * hd;
            for (int i = 0; i < rot; i++) {
                const float ang = (float)pos2[2 * (size_t)p + (i < quarter ? 0 : 1)] * inv_freq[i < quarter ? i : i - quarter];
                const REAL c = cos((REAL)ang), s = sin((REAL)ang);
                for (int part = 0; part < 2; part++) {
                    const int base = part * E + h * hd;
                    const REAL x0 = (REAL)row[base + i] + (bias ? (REAL)bias[base + i] : 0);
                    const REAL x1 = (REAL)row[base + i + rot] + (bias ? (REAL)bias[base + i + rot] : 0);
                    REAL *dst = part == 0 ? Q : K;
                    dst[o + i] = x0 * c - x1 * s;
                    dst[o + i + rot] = x1 * c + x0 * s;
                }
                const int vb = 2 * E + h * hd;
                V[o + i] = (REAL)row[vb + i] + (bias ? (REAL)bias[vb + i] : 0);
                V[o + i + rot] = (REAL)row[vb + i + rot] + (bias ? (REAL)bias[vb + i + rot] : 0);
            }
        }
    }
}

/* metal/clef.metal:2074-2131 (omni_attn_prep) as tests/test_omni_attention.m:104-122 checks it:
 * qkv [T][(nh + 2 nkv) * 128] f32 holds [nh Q] [nkv K] [nkv V]; per head RMSNorm with the weights
 * as given, then rotary over all 64 pairs (i, i + 64), pair i by pos3 axis i % 3 for i < 60 and
 * axis 0 for the last four. exact != 0: angle = pos * theta^(-2i/128) in REAL; exact == 0: the
 * f32 product (float)pos * inv_freq[i]. Q [nh][T][128], K / V [nkv][T][128]. */
void SFX(orc_omni_prep)(int T, int nh, int nkv, double eps, int exact, double theta,
                        const float *qkv, const float *qnorm, const float *knorm,
                        const int32_t *pos3, const float *inv_freq, REAL *Q, REAL *K, REAL *V) {
    const int hd = 128, row = (nh + 2 * nkv) * hd;
#pragma omp parallel for collapse(2) schedule(static)
    for (int t = 0; t < T; t++) {
        for (int head = 0; head < nh + nkv; head++) {
            const float *src = qkv + (size_t)t * row + (size_t)head * hd;
            const int is_q = head < nh, kh = head - nh;
            const float *w = is_q ? qnorm : knorm;
            REAL *dst = is_q ? Q + ((size_t)head * T + t) * hd : K + ((size_t)kh * T + t) * hd;
            REAL ss = 0;
            for (int d = 0; d < hd; d++) ss += (REAL)src[d] * (REAL)src[d];
            const REAL inv = (REAL)1 / sqrt(ss / (REAL)hd + (REAL)eps);
            for (int d = 0; d < hd; d++) dst[d] = (REAL)src[d] * inv * (REAL)w[d];
            for (int i = 0; i < 64; i++) {
                const int position = pos3[3 * (size_t)t + (i < 60 ? i % 3 : 0)];
                const REAL ang = exact ? (REAL)((double)position * pow(theta, -2.0 * i / 128.0))
                                       : (REAL)((float)position * inv_freq[i]);
                const REAL c = cos(ang), s = sin(ang);
                const REAL x0 = dst[i], x1 = dst[i + 64];
                dst[i] = x0 * c - x1 * s;
                dst[i + 64] = x1 * c + x0 * s;
            }
            if (!is_q) {
                const float *vs = qkv + (size_t)t * row + (size_t)(nh + nkv + kh) * hd;
                for (int d = 0; d < hd; d++) V[((size_t)kh * T + t) * hd + d] = (REAL)vs[d];
            }
        }
    }
}
