/* CPU restatement of the reference's token selection -- TEST INFRASTRUCTURE
 * ONLY (linked into liboracle.so next to relux_oracle.c).
 *
 *   orc_greedy       Sampler.Greedy            sampler.go:56-68
 *   orc_sample       Sampler.Sample            sampler.go:73-210 (+ 213-262,
 *                    266-282, 286-301)
 *   orc_spec_accept  acceptPhase + resampleRejected + softmaxAlloc
 *                                              speculative.go:203-290, 344-368
 *
 * Every f32 operation is done in the reference's order (sequential sums over
 * the vocabulary in index order, the selection sorts of argsortDescF32 and
 * kthLargest, f32 division by the temperature, multiplication by f32(1/sum)).
 * The one change: each draw of rng.Float32() is an argument (`r`, or the
 * array `u` consumed in draw order), so the device path can be fed the same
 * numbers.  fastexp32 is orc_fastexp32 (mha.go:823-833).
 *
 * What pins these functions (tests/test_sampling.py): the reference's
 * sampler_test.go cases (argmax, first argmax on ties, T -> 0 gives the
 * argmax, top-2 samples only the two largest), plus brute-force
 * constructions that fix each stage: with r swept over [0, 1) the empirical
 * frequencies equal the stated distribution (softmax / top-k / top-p / min-p
 * renormalised), penalties match hand-computed logits, acceptance rates of
 * the speculative test equal min(1, p_t/p_d) and the resample distribution
 * equals norm(max(0, p_t - p_d)).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

float orc_fastexp32(float x);

/* sampler.go:213-262 -- repeat / frequency / presence penalties over the
 * window (the last `window` tokens when window > 0), on distinct tokens. */
static void apply_penalties(float *s, int n, const int *prev, int n_prev, int window, float rp,
                            float fp, float pp) {
    if (n_prev <= 0) return;
    const int *w = prev;
    int nw = n_prev;
    if (window > 0 && n_prev > window) {
        w = prev + (n_prev - window);
        nw = window;
    }
    int *freq = calloc((size_t)n, sizeof(int));
    for (int i = 0; i < nw; i++)
        if (w[i] >= 0 && w[i] < n) freq[w[i]]++;
    for (int tok = 0; tok < n; tok++) {
        if (!freq[tok]) continue;
        if (rp != 1.0f && rp != 0.0f) {
            if (s[tok] > 0)
                s[tok] /= rp;
            else
                s[tok] *= rp;
        }
        if (fp != 0.0f) {
            volatile float t = fp * (float)freq[tok];
            s[tok] -= t;
        }
        if (pp != 0.0f) s[tok] -= pp;
    }
    free(freq);
}

/* sampler.go:286-301 -- k-th largest by partial selection sort. */
static float kth_largest(const float *a, int n, int k) {
    float *cp = malloc((size_t)n * sizeof(float));
    memcpy(cp, a, (size_t)n * sizeof(float));
    for (int i = 0; i < k; i++) {
        int mj = i;
        for (int j = i + 1; j < n; j++)
            if (cp[j] > cp[mj]) mj = j;
        float t = cp[i];
        cp[i] = cp[mj];
        cp[mj] = t;
    }
    float r = cp[k - 1];
    free(cp);
    return r;
}

static void renormalise(float *p, int n) {
    float sum = 0.0f;
    for (int i = 0; i < n; i++) sum += p[i];
    if (sum > 0) {
        float inv = 1.0f / sum;
        for (int i = 0; i < n; i++) p[i] *= inv;
    }
}

int orc_greedy(const float *logits, int n) {
    int best = 0;
    float bv = logits[0];
    for (int i = 1; i < n; i++)
        if (logits[i] > bv) {
            bv = logits[i];
            best = i;
        }
    return best;
}

/* fparams: temperature, top_p, min_p, repeat_penalty, frequency_penalty,
 * presence_penalty; iparams: top_k, repeat_window.  probs_out (may be NULL)
 * receives the final distribution the draw is taken from. */
int orc_sample(const float *logits, int n, const float *fparams, const int *iparams,
               const int *prev, int n_prev, float r, float *probs_out) {
    float *s = malloc((size_t)n * sizeof(float));
    float *p = malloc((size_t)n * sizeof(float));
    memcpy(s, logits, (size_t)n * sizeof(float));
    apply_penalties(s, n, prev, n_prev, iparams[1], fparams[3], fparams[4], fparams[5]);
    float temp = fparams[0];
    if (temp <= 0) temp = 1e-5f;
    if (temp != 1.0f)
        for (int i = 0; i < n; i++) s[i] /= temp;
    int top_k = iparams[0];
    if (top_k < 0) top_k = 0;
    if (top_k >= n) top_k = 0;
    if (top_k > 0) {
        float thr = kth_largest(s, n, top_k);
        for (int i = 0; i < n; i++)
            if (s[i] < thr) s[i] = -INFINITY;
    }
    float mx = s[0];
    for (int i = 1; i < n; i++)
        if (s[i] > mx) mx = s[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        if (isinf(s[i]) && s[i] < 0) {
            p[i] = 0;
        } else {
            p[i] = orc_fastexp32(s[i] - mx);
            sum += p[i];
        }
    }
    if (sum > 0) {
        float inv = 1.0f / sum;
        for (int i = 0; i < n; i++) p[i] *= inv;
    }
    float top_p = fparams[1];
    if (top_p <= 0 || top_p > 1) top_p = 1.0f;
    if (top_p < 1.0f) {
        /* argsortDescF32's selection sort, run only as far as the cutoff
         * (its prefix does not depend on the later steps). */
        int *idx = malloc((size_t)n * sizeof(int));
        for (int i = 0; i < n; i++) idx[i] = i;
        float cum = 0.0f;
        int cutoff = n;
        for (int i = 0; i < n; i++) {
            int mj = i;
            for (int j = i + 1; j < n; j++)
                if (p[idx[j]] > p[idx[mj]]) mj = j;
            int t = idx[i];
            idx[i] = idx[mj];
            idx[mj] = t;
            cum += p[idx[i]];
            if (cum >= top_p) {
                cutoff = i + 1;
                break;
            }
        }
        for (int j = cutoff; j < n; j++) p[idx[j]] = 0;
        free(idx);
        renormalise(p, n);
    }
    float min_p = fparams[2];
    if (min_p > 0) {
        float mp = 0.0f;
        for (int i = 0; i < n; i++)
            if (p[i] > mp) mp = p[i];
        float thr = mp * min_p;
        for (int i = 0; i < n; i++)
            if (p[i] < thr) p[i] = 0;
        renormalise(p, n);
    }
    float cum = 0.0f;
    int result = n - 1;
    for (int i = 0; i < n; i++) {
        cum += p[i];
        if (r < cum) {
            result = i;
            break;
        }
    }
    if (probs_out) memcpy(probs_out, p, (size_t)n * sizeof(float));
    free(s);
    free(p);
    return result;
}

/* speculative.go:344-368 -- softmax with fastexp32, no -inf test. */
static void softmax_alloc(const float *x, int n, float *p) {
    float mx = x[0];
    for (int i = 1; i < n; i++)
        if (x[i] > mx) mx = x[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        p[i] = orc_fastexp32(x[i] - mx);
        sum += p[i];
    }
    if (sum > 0) {
        float inv = 1.0f / sum;
        for (int i = 0; i < n; i++) p[i] *= inv;
    }
}

/* speculative.go:247-290 -- sample norm(max(0, t - d)); t if that is empty. */
static int resample_rejected(const float *dp, const float *tp, int n, float r) {
    float *adj = malloc((size_t)n * sizeof(float));
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        float d = tp[i] - dp[i];
        if (d < 0) d = 0;
        adj[i] = d;
        sum += d;
    }
    int result = 0;
    float cum = 0.0f;
    if (sum > 0) {
        float inv = 1.0f / sum;
        for (int i = 0; i < n; i++) {
            volatile float t = adj[i] * inv;
            cum += t;
            if (r < cum) {
                result = i;
                break;
            }
        }
    } else {
        for (int i = 0; i < n; i++) {
            cum += tp[i];
            if (r < cum) {
                result = i;
                break;
            }
        }
    }
    free(adj);
    return result;
}

/* speculative.go:203-244.  d_logits [k][n], t_logits [k+1][n], u [k+1]:
 * u[i] is the acceptance draw of draft i; the draw after the last test
 * feeds resample_rejected or the final Sample.  Returns the accepted count;
 * *next = the resampled (or, all accepted, sampled) token. */
int orc_spec_accept(const float *d_logits, const float *t_logits, const int *d_tok, int k, int n,
                    const float *u, const float *fparams, const int *iparams, int *next) {
    float *dp = malloc((size_t)n * sizeof(float));
    float *tp = malloc((size_t)n * sizeof(float));
    int draw = 0;
    for (int i = 0; i < k; i++) {
        softmax_alloc(d_logits + (int64_t)i * n, n, dp);
        softmax_alloc(t_logits + (int64_t)i * n, n, tp);
        float dP = dp[d_tok[i]], tP = tp[d_tok[i]];
        float a = tP / (dP > 1e-10f ? dP : 1e-10f);
        if (a > 1) a = 1;
        if (u[draw++] < a) continue;
        *next = resample_rejected(dp, tp, n, u[draw]);
        free(dp);
        free(tp);
        return i;
    }
    const int no_prev_i[2] = {iparams[0], 0};
    *next = orc_sample(t_logits + (int64_t)k * n, n, fparams, no_prev_i, NULL, 0, u[draw], NULL);
    free(dp);
    free(tp);
    return k;
}
