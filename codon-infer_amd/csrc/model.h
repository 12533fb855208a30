// Device-resident model and workspace (shared by the forward, the loader and
// the utility entry points).  Internal, not part of the C ABI.
#pragma once
#include <hip/hip_runtime.h>

#include <string>
#include <vector>

#include "host.h"
#include "kernels.h"

#define HIPCHK(expr)                                                                                     \
    do {                                                                                                 \
        hipError_t e_ = (expr);                                                                          \
        if (e_ != hipSuccess) return set_error(CIH_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

namespace cih {

struct Layer {
    DevMatrix wqkv, wo, w1, w2;
    float *bqkv = nullptr, *bo = nullptr, *b1 = nullptr, *b2 = nullptr;
    float *ln1w = nullptr, *ln1b = nullptr, *ln2w = nullptr, *ln2b = nullptr;
};

// What fixes a forward's kernel sequence: grids, pointers, and the kernel
// switches read while it is enqueued (kernel_switches()).
struct FwdGraphKey {
    // tiles: sum over sequences of ceil(len / 32), the grid of the K/V image
    // prep kernel; lengths with the same B, S_max and T can differ in it
    int B = 0, S_max = 0, T = 0, tiles = 0;
    uint32_t flags = 0;
    const void *out[6] = {};
    std::string sw;
    bool operator==(const FwdGraphKey &o) const {
        if (B != o.B || S_max != o.S_max || T != o.T || tiles != o.tiles || flags != o.flags || sw != o.sw)
            return false;
        for (int i = 0; i < 6; i++)
            if (out[i] != o.out[i]) return false;
        return true;
    }
};

struct Workspace {
    int maxB = 0, maxS = 0;
    uint32_t flags = 0;
    int *tokens = nullptr, *cu = nullptr, *lens = nullptr;
    int *h_meta = nullptr;  // pinned: cu[maxB] | lens[maxB] | status word read back
    int *flag = nullptr;    // device status word of the forward (FLAG_* bits)
    float *x = nullptr, *xb = nullptr, *qkv = nullptr, *ao = nullptr, *hbuf = nullptr, *logits = nullptr;
    float *rope_c = nullptr, *rope_s = nullptr;
    float *P = nullptr;                            // [maxB][H][maxS][maxS] probabilities scratch
    float *M = nullptr, *r = nullptr, *coef = nullptr;  // contacts
    float *rowsum = nullptr, *colpart = nullptr;        // contacts: map row sums, column partial sums
    PartialBuf part;                                    // partial sums of k-split GEMMs / GEMVs
    float *attp = nullptr;                              // partial results of key-split attention
    size_t attp_floats = 0;
    // K/V tile images (kv_image.h) written by the QKV projection's epilogue
    unsigned char *kv_img = nullptr;
    int *kv_tb = nullptr, *kv_pk = nullptr, *kv_pos = nullptr;  // [maxB], [T], [T]
    int *kv_ti = nullptr;  // [tile rows][4]: first packed row, keys, first position, sequence
    int *dms_meta = nullptr;                            // [max(maxB, maxS)][2] scored row, wild type
    float *dms_out = nullptr;                           // [max(maxB, maxS)][21] deltas, entropy
    // device staging of outputs for host-pointer calls (padded layouts)
    float *o_logits = nullptr, *o_hidden = nullptr, *o_final = nullptr, *o_contacts = nullptr, *o_attn = nullptr,
          *o_layer = nullptr;
    // pinned host staging of those outputs on their way to the caller's
    // (pageable) buffers: blocks of whole rows, h_stage_floats at a time
    float *h_stage = nullptr;
    size_t h_stage_floats = 0;
    std::vector<void *> dev, host;
    // captured forwards, by shape
    std::vector<std::pair<FwdGraphKey, hipGraphExec_t>> graphs;
};

struct Prof {
    bool on = false;
    std::vector<hipEvent_t> ev;  // pairs
    std::vector<int> cls;
    std::vector<double> flops, bytes;
    size_t used = 0;
    cih_kernel_stats st[CIH_KC_COUNT] = {};
};

}  // namespace cih

struct cih_model {
    cih_config cfg{};
    int dtype = 0, hd = 0;
    int device = 0;
    hipStream_t stream = nullptr;
    std::vector<void *> allocs;
    cih::DevMatrix emb;
    std::vector<cih::Layer> layers;
    float *lnfw = nullptr, *lnfb = nullptr;
    bool has_head = false;
    cih::DevMatrix dense, dec;
    float *dense_b = nullptr, *lm_lnw = nullptr, *lm_lnb = nullptr, *dec_b = nullptr;
    std::vector<float> contact_w;
    float contact_b = 0.0f;
    bool has_contacts = false;
    float *d_contact_w = nullptr;
    int *d_heads = nullptr;  // [L][H] per-layer list of heads with nonzero weight
    std::vector<int> nz;
    cih::Workspace ws;
    cih::Prof prof;
};

namespace cih {

template <class T>
hipError_t dalloc(T *&p, size_t n, std::vector<void *> &list) {
    p = nullptr;
    if (n == 0) return hipSuccess;
    void *v = nullptr;
    hipError_t e = hipMalloc(&v, n * sizeof(T));
    if (e != hipSuccess) return e;
    list.push_back(v);
    p = (T *)v;
    return hipSuccess;
}

template <class T>
int upload(cih_model *m, T *&dst, const T *src, size_t n) {
    HIPCHK(dalloc(dst, n, m->allocs));
    if (n) HIPCHK(hipMemcpy(dst, src, n * sizeof(T), hipMemcpyHostToDevice));
    return 0;
}

// Records an event pair around the launches of its scope on the model's
// stream when profiling is on (class, algorithmic flops and bytes).
struct ProfScope {
    cih_model *m;
    int idx = -1;
    ProfScope(cih_model *m_, int cls, double flops, double bytes) : m(m_) {
        Prof &p = m->prof;
        if (!p.on) return;
        if (p.used >= p.cls.size()) {
            hipEvent_t a, b;
            if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) return;
            p.ev.push_back(a);
            p.ev.push_back(b);
            p.cls.push_back(0);
            p.flops.push_back(0);
            p.bytes.push_back(0);
        }
        idx = (int)p.used++;
        p.cls[idx] = cls;
        p.flops[idx] = flops;
        p.bytes[idx] = bytes;
        hipEventRecord(p.ev[2 * idx], m->stream);
    }
    ~ProfScope() {
        if (idx >= 0) hipEventRecord(m->prof.ev[2 * idx + 1], m->stream);
    }
};

void free_list(std::vector<void *> &l);
int check_config(const cih_config *c);

// The values of the environment switches that choose kernels while a
// forward or decode step is enqueued, plus full-range mode: part of the key
// of a captured graph, so that a change of switch is never hidden by the
// replay of a graph captured under other settings.
std::string kernel_switches();

// Runs fn() with full-range mode on for this thread (full_range_mode()).
void set_full_range_mode(bool on);
template <class F>
int in_full_range(F fn) {
    set_full_range_mode(true);
    const int rc = fn();
    set_full_range_mode(false);
    return rc;
}

// algorithmic bytes of a weight matrix
double wbytes(const DevMatrix &W);
// A few FP32 rows go to the weight-streaming GEMV (CIH_GEMV=0 turns it off).
bool use_gemv(int M, int a_fmt, int epi);

// Y = epi(X W^T + bias) on the model's stream: the weight-streaming GEMV for
// a few FP32 rows, the MFMA GEMM otherwise; partial sums through pb.
hipError_t model_gemm(cih_model *m, const PartialBuf &pb, const DevMatrix &W, const void *X, int ldx, int a_fmt,
                      const float *bias, void *Y, int ldy, int M, int epi, int *defer = nullptr);
// After the stream has drained: adds the launches recorded since the last
// call (event pairs of model_gemm and friends) to the per-class totals.
void profile_collect(cih_model *m);
// partial-sum floats any GEMM / GEMV of the model needs
// partial-sum floats a workspace for `tokens` tokens needs (split GEMMs and GEMVs)
size_t model_part_floats(const cih_model *m, size_t tokens = 0);
// RoPE cos / sin tables [max_len][hd/2] as the reference computes them
void rope_tables_host(size_t max_len, int hd, std::vector<float> &c, std::vector<float> &s);

// One [N][K] host matrix (FP32 values or reference row-major blocks) that
// becomes rows [n_off, n_off + N) of a device matrix.
struct Part {
    const void *src;
    int N;
};

// Builds a device matrix in the k-block-major layout from host parts of
// dtype src_dt (one H2D copy, repack on the GPU), stored as dst_dt: equal to
// src_dt, or Q8_0 / Q4_0 quantized on the GPU from FP32.  Buffers go to
// m->allocs.
// pair: FP32 destinations also get the f16 pair copy (CIH_F32_PAIR=0: never)
int upload_matrix(cih_model *m, int src_dt, int dst_dt, int K, const std::vector<Part> &parts, DevMatrix &out,
                  bool pair = false);

}  // namespace cih
