/*
 * pipeline.c — a C caller of include/codon_hip.h that runs the two call
 * sequences of codon-infer's pipeline.rs on the GPU library, the way a host
 * program drives it without Python:
 *
 *   contacts: compute_pipeline_contacts_parallel (src/pipeline.rs:410-513):
 *             load, Tokenizer::encode, one forward with contacts, then the
 *             pairs at separation >= min_sep sorted by probability (stable,
 *             descending), top_k = max_k or clamp(round(n * top_l_factor),
 *             5, 50), and the Cys-Cys enrichment of the top pairs.
 *   dms:      run_pipeline_dms_with_mode (src/pipeline.rs:76-315) through
 *             cih_dms, then DmsPositionRow::new per position (src/export.rs:
 *             17-40: mean of the non-zero deltas over 19, category) and the
 *             count of positions with mean <= -3.8.
 *
 * Usage:
 *   pipeline contacts <weights> <contact_head.bin> <sequence> <min_sep> <top_l_factor> <max_k|0> <map.bin>
 *   pipeline dms <weights> <sequence> <window> <stride> <mode 0|1> <chunk>
 * <weights>: a CODQ / grouped_canonical_v1 / sequential_hf file;
 * <contact_head.bin>: n_layers * n_heads float32 regression weights, then
 * the float32 bias.  Results go to stdout as text lines; the contact map is
 * also written to <map.bin> as n * n float32.  Exit status 0 on success,
 * else 1 with the library's error on stderr.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "../../include/codon_hip.h"

static int fail(const char *what, int rc) {
    fprintf(stderr, "%s failed (%d): %s\n", what, rc, cih_last_error());
    return 1;
}

static double now_ms(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e3 + ts.tv_nsec * 1e-6;
}

typedef struct {
    int i, j;
    float score;
    int order; /* position in the (i, j) scan: keeps the sort stable */
} pair_t;

/* descending score; equal scores keep their scan order (a stable sort) */
static int by_score(const void *a, const void *b) {
    const pair_t *x = (const pair_t *)a, *y = (const pair_t *)b;
    if (x->score > y->score) return -1;
    if (x->score < y->score) return 1;
    return x->order - y->order;
}

static int run_contacts(int argc, char **argv) {
    if (argc != 9) {
        fprintf(stderr, "usage: pipeline contacts <weights> <contact_head.bin> <sequence> <min_sep> "
                        "<top_l_factor> <max_k|0> <map.bin>\n");
        return 2;
    }
    const char *wpath = argv[2], *cpath = argv[3], *seq = argv[4], *map_path = argv[8];
    const int min_sep = atoi(argv[5]), max_k = atoi(argv[7]);
    const float top_l_factor = (float)atof(argv[6]);
    const int n = (int)strlen(seq);
    if (n < 4) {
        fprintf(stderr, "sequence too short for contact prediction\n");
        return 2;
    }
    /* the contact head: L * H weights and the bias */
    FILE *f = fopen(cpath, "rb");
    if (!f) {
        fprintf(stderr, "cannot open %s\n", cpath);
        return 1;
    }
    float buf[4096];
    const size_t got = fread(buf, sizeof(float), 4096, f);
    fclose(f);
    if (got < 2) {
        fprintf(stderr, "%s: too short\n", cpath);
        return 1;
    }
    cih_model *m = NULL;
    int rc = cih_model_create_from_file(wpath, -1, buf, buf[got - 1], &m);
    if (rc) return fail("cih_model_create_from_file", rc);
    cih_config cfg;
    int32_t dtype = 0;
    cih_model_config(m, &cfg, &dtype);
    if ((int)got != cfg.n_layers * cfg.n_heads + 1) {
        fprintf(stderr, "%s: %zu floats, expected %d\n", cpath, got, cfg.n_layers * cfg.n_heads + 1);
        cih_model_destroy(m);
        return 1;
    }
    int32_t *tokens = (int32_t *)malloc(sizeof(int32_t) * (n + 2));
    const int S = cih_tokenize(seq, tokens, n + 2);
    if (S != n + 2) {
        cih_model_destroy(m);
        return fail("cih_tokenize", S);
    }
    if ((rc = cih_model_reserve(m, 1, S, CIH_OUT_CONTACTS))) {
        cih_model_destroy(m);
        return fail("cih_model_reserve", rc);
    }
    float *probs = (float *)malloc(sizeof(float) * (size_t)n * n);
    cih_outputs out;
    memset(&out, 0, sizeof out);
    out.contacts = probs;
    const int32_t len = S;
    const double t0 = now_ms();
    rc = cih_forward(m, tokens, &len, 1, S, CIH_OUT_CONTACTS, &out);
    const double t1 = now_ms();
    cih_model_destroy(m);
    if (rc) return fail("cih_forward", rc);

    /* candidate pairs in the reference's scan order, Cys statistics */
    int n_cys = 0, cys_pairs = 0, total = 0;
    for (int i = 0; i < n; i++) n_cys += seq[i] == 'C';
    const long max_pairs = (long)n * n / 2 + n;
    pair_t *pairs = (pair_t *)malloc(sizeof(pair_t) * max_pairs);
    int np = 0;
    for (int i = 0; i < n; i++)
        for (int j = i + min_sep; j < n; j++) {
            const int cc = seq[i] == 'C' && seq[j] == 'C';
            total++;
            cys_pairs += cc;
            pairs[np].i = i;
            pairs[np].j = j;
            pairs[np].score = probs[(size_t)i * n + j];
            pairs[np].order = np;
            np++;
        }
    qsort(pairs, np, sizeof(pair_t), by_score);
    int top_k;
    if (max_k > 0) {
        top_k = max_k < np ? max_k : np;
    } else {
        int k = (int)roundf((float)n * top_l_factor);
        k = k < 5 ? 5 : (k > 50 ? 50 : k);
        top_k = k < np ? k : np;
    }
    int top_cys = 0;
    for (int t = 0; t < top_k; t++) top_cys += seq[pairs[t].i] == 'C' && seq[pairs[t].j] == 'C';
    const float top_density = top_k > 0 ? (float)top_cys / (float)top_k : 0.0f;
    const float bg_density = total > 0 ? (float)cys_pairs / (float)total : 0.05f;
    const float enrichment = bg_density > 0.0f ? top_density / bg_density : 1.0f;

    printf("n %d\n", n);
    printf("forward_ms %.3f\n", t1 - t0);
    printf("n_cys %d\n", n_cys);
    printf("top_k %d\n", top_k);
    for (int t = 0; t < top_k; t++)
        printf("top %d %c %d %c %.9g %d\n", pairs[t].i, seq[pairs[t].i], pairs[t].j, seq[pairs[t].j], pairs[t].score,
               seq[pairs[t].i] == 'C' && seq[pairs[t].j] == 'C');
    printf("cys_enrichment %.9g\n", enrichment);
    FILE *mf = fopen(map_path, "wb");
    if (!mf || fwrite(probs, sizeof(float), (size_t)n * n, mf) != (size_t)n * n) {
        fprintf(stderr, "cannot write %s\n", map_path);
        if (mf) fclose(mf);
        return 1;
    }
    fclose(mf);
    free(pairs);
    free(probs);
    free(tokens);
    return 0;
}

static const char CANONICAL[] = "ACDEFGHIKLMNPQRSTVWY"; /* CANONICAL_AAS order, benchmark.rs:702-707 */

static int run_dms(int argc, char **argv) {
    if (argc != 8) {
        fprintf(stderr, "usage: pipeline dms <weights> <sequence> <window> <stride> <mode 0|1> <chunk>\n");
        return 2;
    }
    const char *wpath = argv[2], *seq = argv[3];
    const int window = atoi(argv[4]), stride = atoi(argv[5]), mode = atoi(argv[6]), chunk = atoi(argv[7]);
    const int n = (int)strlen(seq);
    if (n < 1) {
        fprintf(stderr, "sequence cannot be empty\n");
        return 2;
    }
    cih_model *m = NULL;
    int rc = cih_model_create_from_file(wpath, -1, NULL, 0.0f, &m);
    if (rc) return fail("cih_model_create_from_file", rc);
    cih_config cfg;
    int32_t dtype = 0;
    cih_model_config(m, &cfg, &dtype);
    /* BidirectionalRunState::new(config, actual_window + 2), pipeline.rs:90-96 */
    const int aw = (n <= window || window == 0) ? (n < cfg.max_seq_len ? n : cfg.max_seq_len)
                                                 : (window < cfg.max_seq_len ? window : cfg.max_seq_len);
    const int batch = mode == CIH_DMS_MASKED_MARGINAL ? (chunk > 0 ? chunk : 1) : 1;
    if ((rc = cih_model_reserve(m, batch, aw + 2, 0))) {
        cih_model_destroy(m);
        return fail("cih_model_reserve", rc);
    }
    int32_t *tokens = (int32_t *)malloc(sizeof(int32_t) * (n + 2));
    if (cih_tokenize(seq, tokens, n + 2) != n + 2) {
        cih_model_destroy(m);
        return fail("cih_tokenize", -1);
    }
    float *deltas = (float *)malloc(sizeof(float) * 20 * (size_t)n), *entropy = (float *)malloc(sizeof(float) * n);
    const double t0 = now_ms();
    rc = cih_dms(m, tokens + 1, n, window, stride, mode, chunk, deltas, entropy);
    const double el = now_ms() - t0;
    cih_model_destroy(m);
    if (rc) return fail("cih_dms", rc);
    int catalytic = 0;
    printf("n %d\n", n);
    for (int p = 0; p < n; p++) {
        /* DmsPositionRow::new: the non-zero deltas summed in order, over 19 */
        float sum = 0.0f;
        for (int a = 0; a < 20; a++)
            if (deltas[(size_t)p * 20 + a] != 0.0f) sum += deltas[(size_t)p * 20 + a];
        const float mean = sum / 19.0f;
        const char *cat = mean <= -3.8f ? "catalytic" : (mean <= -2.2f ? "core" : "tolerated");
        catalytic += mean <= -3.8f;
        printf("row %d %c %.9g %.9g %s", p + 1, seq[p], mean, entropy[p], cat);
        for (int a = 0; a < 20; a++) printf(" %.9g", deltas[(size_t)p * 20 + a]);
        printf("\n");
    }
    printf("canonical %s\n", CANONICAL);
    printf("elapsed_ms %.3f\n", el);
    printf("muts_per_sec %.1f\n", el > 0 ? (double)n * 20.0 / (el * 1e-3) : 0.0);
    printf("catalytic_sites %d\n", catalytic);
    free(deltas);
    free(entropy);
    free(tokens);
    return 0;
}

int main(int argc, char **argv) {
    if (argc >= 2 && !strcmp(argv[1], "contacts")) return run_contacts(argc, argv);
    if (argc >= 2 && !strcmp(argv[1], "dms")) return run_dms(argc, argv);
    fprintf(stderr, "usage: pipeline contacts|dms ...\n");
    return 2;
}
