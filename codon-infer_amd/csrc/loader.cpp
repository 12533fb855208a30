// Model residency: weight files and caller-owned host tensors become a
// device-resident model.  The reference's bytes go to the GPU unchanged —
// parallel reads (or copies) into pinned staging buffers, asynchronous H2D
// copies on one stream per staging thread — and the GPU repacks them into
// the k-block-major layout of kernels.h, quantizing FP32 matrices when asked.
// The host never touches a weight value.
//
// Replaces EsmWeights::from_file / EsmWeightsQ8::from_file /
// EsmWeightsQ4::from_file (src/lib.rs:310-547, 744-830, 1156-1242),
// EsmWeights::quantize_q8 / quantize_q4 (lib.rs:559-607) and the CODQ header
// checks (lib.rs:887-1037).
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <atomic>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <thread>

#include "model.h"

namespace cih {
namespace {

// ---- where every tensor sits in a weights body ----------------------------

// EsmConfig presets (lib.rs:86-145) indexed by CODQ arch id (lib.rs:878-882).
const cih_config kPresets[] = {
    {320, 1280, 6, 20, 33, 1024},  {480, 1920, 12, 20, 33, 1024},  {640, 2560, 30, 20, 33, 1024},
    {1280, 5120, 33, 20, 33, 1024}, {2560, 10240, 36, 40, 33, 1024},
};

int64_t lm_head_floats(const cih_config &c) {
    return 3LL * c.dim + (int64_t)c.dim * c.dim + (int64_t)c.vocab_size * c.dim + c.vocab_size;
}

// grouped_canonical_floats (lib.rs:195-204)
int64_t grouped_floats(const cih_config &c) {
    const int64_t d = c.dim, F = c.hidden_dim;
    return (int64_t)c.vocab_size * d + (int64_t)c.n_layers * (4 * d * d + 9 * d + 2 * d * F + F) + 2 * d +
           lm_head_floats(c);
}

// sequential_hf_floats (lib.rs:212-218): + rotary inv_freq + contact head
int64_t sequential_floats(const cih_config &c) {
    return grouped_floats(c) + (c.dim / c.n_heads) / 2 + (int64_t)c.n_layers * c.n_heads + 1;
}

int64_t mat_bytes(int dtype, int64_t elems) { return dtype == DT_FP32 ? elems * 4 : elems / 32 * block_bytes(dtype); }

// Byte offsets of the tensors in a weights body (per layer where stacked).
// Matrices are stored in `dtype` (FP32 values or packed blocks), the token
// embedding in emb_dtype, everything else in FP32.
struct Layout {
    int dtype = DT_FP32, emb_dtype = DT_FP32;
    int64_t emb = 0;
    std::vector<int64_t> ln1w, ln1b, wq, bq, wk, bk, wv, bv, wo, bo, ln2w, ln2b, fc1, fc1b, fc2, fc2b;
    int64_t lnfw = 0, lnfb = 0;
    bool head = false;  // LM head present: [ln_w, ln_b, dense_w, dense_b, dec_w, dec_b]
    int64_t lm_lnw = 0, lm_lnb = 0, dense_w = 0, dense_b = 0, dec_w = 0, dec_b = 0;
    int64_t total = 0;
};

// Tensor-major bodies: grouped_canonical_v1 (lib.rs:369-395) and the
// EsmWeightsQ8/Q4 save order (lib.rs:716-742, 1128-1154), which is the same
// with blocks for the matrices (and a Q8_0 embedding for Q8_0); the
// classifier is whatever floats remain (cls_floats).
Layout grouped_layout(const cih_config &c, int dtype, int64_t cls_floats) {
    const int64_t d = c.dim, F = c.hidden_dim, L = c.n_layers, V = c.vocab_size;
    Layout y;
    y.dtype = dtype;
    y.emb_dtype = dtype == DT_Q8 ? DT_Q8 : DT_FP32;
    int64_t off = 0;
    auto field = [&](std::vector<int64_t> &v, int64_t per_layer) {
        v.resize(L);
        for (int64_t l = 0; l < L; l++) v[l] = off + l * per_layer;
        off += L * per_layer;
    };
    y.emb = off;
    off += mat_bytes(y.emb_dtype, V * d);
    field(y.ln1w, 4 * d);
    field(y.ln1b, 4 * d);
    field(y.wq, mat_bytes(dtype, d * d));
    field(y.bq, 4 * d);
    field(y.wk, mat_bytes(dtype, d * d));
    field(y.bk, 4 * d);
    field(y.wv, mat_bytes(dtype, d * d));
    field(y.bv, 4 * d);
    field(y.wo, mat_bytes(dtype, d * d));
    field(y.bo, 4 * d);
    field(y.ln2w, 4 * d);
    field(y.ln2b, 4 * d);
    field(y.fc1, mat_bytes(dtype, F * d));
    field(y.fc1b, 4 * F);
    field(y.fc2, mat_bytes(dtype, d * F));
    field(y.fc2b, 4 * d);
    y.lnfw = off;
    y.lnfb = off + 4 * d;
    off += 8 * d;
    y.head = cls_floats >= lm_head_floats(c);
    y.lm_lnw = off;
    y.lm_lnb = off + 4 * d;
    y.dense_w = off + 8 * d;
    y.dense_b = y.dense_w + 4 * d * d;
    y.dec_w = y.dense_b + 4 * d;
    y.dec_b = y.dec_w + 4 * V * d;
    y.total = off + 4 * cls_floats;
    return y;
}

// sequential_hf (lib.rs:396-499): embedding, rotary inv_freq, then per layer
// wq bq wk bk wv bv wo bo ln1w ln1b fc1 fc1b fc2 fc2b ln2w ln2b, then lnf_w,
// lnf_b, the contact head (L*H + 1), lm bias, dense_w, dense_b, lm ln_w,
// lm ln_b, decoder_w.
Layout sequential_layout(const cih_config &c) {
    const int64_t d = c.dim, F = c.hidden_dim, L = c.n_layers, V = c.vocab_size;
    Layout y;
    int64_t off = 4 * V * d + 4 * ((d / c.n_heads) / 2);
    for (auto *v : {&y.ln1w, &y.ln1b, &y.wq, &y.bq, &y.wk, &y.bk, &y.wv, &y.bv, &y.wo, &y.bo, &y.ln2w, &y.ln2b,
                    &y.fc1, &y.fc1b, &y.fc2, &y.fc2b})
        v->resize(L);
    for (int64_t l = 0; l < L; l++) {
        auto put = [&](std::vector<int64_t> &v, int64_t floats) {
            v[l] = off;
            off += 4 * floats;
        };
        put(y.wq, d * d); put(y.bq, d); put(y.wk, d * d); put(y.bk, d); put(y.wv, d * d); put(y.bv, d);
        put(y.wo, d * d); put(y.bo, d); put(y.ln1w, d); put(y.ln1b, d); put(y.fc1, F * d); put(y.fc1b, F);
        put(y.fc2, d * F); put(y.fc2b, d); put(y.ln2w, d); put(y.ln2b, d);
    }
    y.lnfw = off;
    y.lnfb = off + 4 * d;
    off += 8 * d + 4 * ((int64_t)L * c.n_heads + 1);
    y.head = true;
    y.dec_b = off;
    off += 4 * V;
    y.dense_w = off;
    off += 4 * d * d;
    y.dense_b = off;
    off += 4 * d;
    y.lm_lnw = off;
    y.lm_lnb = off + 4 * d;
    off += 8 * d;
    y.dec_w = off;
    y.total = off + 4 * V * d;
    return y;
}

// ---- file header and size checks (errors as EsmWeights*::from_file) -------

struct FileInfo {
    cih_config cfg{};
    Layout layout;
    int64_t body_off = 0;
};

struct Fd {
    int fd = -1;
    ~Fd() {
        if (fd >= 0) close(fd);
    }
};

bool read_at(int fd, void *dst, int64_t n, int64_t off) {
    uint8_t *p = (uint8_t *)dst;
    while (n > 0) {
        const ssize_t r = pread(fd, p, (size_t)n, (off_t)off);
        if (r <= 0) return false;
        p += r;
        off += r;
        n -= r;
    }
    return true;
}

int fp32_body(const cih_config &c, int64_t remaining, Layout &y) {
    if (remaining % 4) return set_error(CIH_ERR_FORMAT, "unaligned trailing bytes: %lld", (long long)remaining);
    const int64_t nf = remaining / 4;
    if (nf == grouped_floats(c)) {
        y = grouped_layout(c, DT_FP32, lm_head_floats(c));
        return 0;
    }
    if (nf == sequential_floats(c)) {
        y = sequential_layout(c);
        return 0;
    }
    return set_error(CIH_ERR_FORMAT,
                     "invalid FP32 weights size: %lld floats, expected %lld (grouped_canonical_v1) or %lld "
                     "(sequential_hf)",
                     (long long)nf, (long long)grouped_floats(c), (long long)sequential_floats(c));
}

int parse_file(const char *path, int fd, FileInfo &fi) {
    struct stat sb;
    if (fstat(fd, &sb) != 0) return set_error(CIH_ERR_IO, "cannot stat %s", path);
    const int64_t flen = sb.st_size;
    unsigned char hdr[64] = {0};
    const bool has_hdr = flen >= 64 && read_at(fd, hdr, 64, 0) && !std::memcmp(hdr, "CODQ", 4);
    if (has_hdr) {
        // CodqHeader (lib.rs:887-898): magic, version, dtype, arch, n_layers, dim, hidden, vocab, 32 reserved
        uint32_t h[8];
        std::memcpy(h, hdr, 32);
        if (h[1] != 1) return set_error(CIH_ERR_FORMAT, "unsupported CODQ version %u", h[1]);
        if (h[3] > 4) return set_error(CIH_ERR_FORMAT, "unknown CODQ arch id %u", h[3]);
        const cih_config &c = kPresets[h[3]];
        if ((int)h[4] != c.n_layers || (int)h[5] != c.dim || (int)h[6] != c.hidden_dim || (int)h[7] != c.vocab_size)
            return set_error(CIH_ERR_FORMAT, "incoherent CODQ dimensions for arch %u", h[3]);
        fi.cfg = c;
        fi.body_off = 64;
        const int64_t remaining = flen - 64;
        if (h[2] == DT_FP32) return fp32_body(c, remaining, fi.layout);
        if (h[2] == DT_Q8 || h[2] == DT_Q4) {
            const int dt = (int)h[2];
            const Layout no_cls = grouped_layout(c, dt, 0);
            if (no_cls.total > remaining) return set_error(CIH_ERR_IO, "short read in quantized weights body");
            const int64_t rest = remaining - no_cls.total;
            if (rest % 4) return set_error(CIH_ERR_FORMAT, "unaligned trailing bytes: %lld", (long long)rest);
            fi.layout = grouped_layout(c, dt, rest / 4);
            return 0;
        }
        return set_error(CIH_ERR_FORMAT, "unsupported CODQ dtype %u", h[2]);
    }
    for (const auto &c : kPresets) {
        if (flen == grouped_floats(c) * 4 || flen == sequential_floats(c) * 4) {
            fi.cfg = c;
            fi.body_off = 0;
            return fp32_body(c, flen, fi.layout);
        }
    }
    return set_error(CIH_ERR_FORMAT,
                     "unrecognized weights file %s (%lld bytes): no CODQ header and not an exact FP32 ESM-2 size",
                     path, (long long)flen);
}

// ---- staging: host bytes -> device image ----------------------------------

// `bytes` bytes from host memory (host != nullptr) or from the file at
// file_off, to image offset img_off.
struct Region {
    const uint8_t *host;
    int64_t file_off, img_off, bytes;
};

int env_int(const char *name, int dflt, int lo, int hi) {
    const char *e = getenv(name);
    if (!e || !*e) return dflt;
    const int v = atoi(e);
    return v < lo ? lo : (v > hi ? hi : v);
}

// Each staging thread owns two pinned buffers and a stream: while one
// buffer's copy runs, the thread fills the other.  Chunks are handed out in
// file order, so reads stay nearly sequential.
int stage(int device, int fd, const std::vector<Region> &regs, uint8_t *img) {
    const int64_t chunk = (int64_t)env_int("CIH_LOAD_CHUNK_MB", 8, 1, 256) << 20;
    std::vector<Region> chunks;
    for (const Region &r : regs)
        for (int64_t o = 0; o < r.bytes; o += chunk)
            chunks.push_back({r.host ? r.host + o : nullptr, r.file_off + o, r.img_off + o, std::min(chunk, r.bytes - o)});
    if (chunks.empty()) return 0;
    const int hw = (int)std::max(1u, std::thread::hardware_concurrency());
    const int nt = (int)std::min<int64_t>((int64_t)chunks.size(), env_int("CIH_LOAD_THREADS", std::min(2, hw), 1, 64));
    std::atomic<size_t> next{0};
    std::atomic<bool> failed{false};
    std::mutex mu;
    int err_code = 0;
    std::string err;
    auto fail = [&](int code, const std::string &msg) {
        std::lock_guard<std::mutex> g(mu);
        if (!err_code) {
            err_code = code;
            err = msg;
        }
        failed = true;
    };
    auto hip_fail = [&](const char *what, hipError_t e) { fail(CIH_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e)); };
    auto worker = [&]() {
        hipStream_t st = nullptr;
        uint8_t *buf[2] = {nullptr, nullptr};
        hipEvent_t ev[2] = {nullptr, nullptr};
        hipError_t e = hipSetDevice(device);
        if (e == hipSuccess) e = hipStreamCreate(&st);
        for (int b = 0; b < 2 && e == hipSuccess; b++) {
            e = hipHostMalloc((void **)&buf[b], (size_t)chunk, hipHostMallocDefault);
            if (e == hipSuccess) e = hipEventCreateWithFlags(&ev[b], hipEventDisableTiming);
        }
        if (e != hipSuccess) hip_fail("staging setup", e);
        size_t c;
        for (int k = 0; e == hipSuccess && !failed && (c = next.fetch_add(1)) < chunks.size(); k++) {
            const int b = k & 1;
            if (k >= 2 && (e = hipEventSynchronize(ev[b])) != hipSuccess) {
                hip_fail("staging copy", e);
                break;
            }
            const Region &r = chunks[c];
            if (r.host) {
                std::memcpy(buf[b], r.host, (size_t)r.bytes);
            } else if (!read_at(fd, buf[b], r.bytes, r.file_off)) {
                fail(CIH_ERR_IO, "short read at file offset " + std::to_string(r.file_off));
                break;
            }
            e = hipMemcpyAsync(img + r.img_off, buf[b], (size_t)r.bytes, hipMemcpyHostToDevice, st);
            if (e == hipSuccess) e = hipEventRecord(ev[b], st);
            if (e != hipSuccess) hip_fail("staging copy", e);
        }
        if (st) {
            hipError_t s = hipStreamSynchronize(st);
            if (s != hipSuccess) hip_fail("staging copy", s);
        }
        for (int b = 0; b < 2; b++) {
            if (ev[b]) hipEventDestroy(ev[b]);
            if (buf[b]) hipHostFree(buf[b]);
        }
        if (st) hipStreamDestroy(st);
    };
    std::vector<std::thread> th;
    for (int t = 0; t < nt; t++) th.emplace_back(worker);
    for (auto &t : th) t.join();
    return err_code ? set_error(err_code, "%s", err.c_str()) : 0;
}

// ---- the GPU build of a model from its image --------------------------------

int wfmt(int dtype) { return dtype == DT_Q8 ? WF_Q8 : (dtype == DT_Q4 ? WF_Q4 : WF_F32); }

// FP32 matrices also keep the f16 pair copy (4.25 bytes per weight) for the
// f16-limb GEMM; CIH_F32_PAIR=0 leaves it out (FP32 MFMA only).
bool pair_copies() {
    const char *e = getenv("CIH_F32_PAIR");
    return !(e && !strcmp(e, "0"));
}

// Device buffers are carved from one allocation: plan (sizes, jobs), then
// allocate, then point and launch.
struct Plan {
    struct Job {
        int src_fmt;
        int64_t src;  // image offset of rows [0, N)
        int N, n_off;
        DevMatrix *dst;
    };
    size_t bytes = 0;
    std::vector<std::pair<const void **, size_t>> fix;
    std::vector<Job> jobs;
    std::vector<CopySeg> copies;
    std::vector<DevMatrix *> expand;  // matrices that also get the f16 copy of their quants
    std::vector<DevMatrix *> pairs;   // FP32 matrices that also get the f16 pair copy

    size_t take(size_t b) {
        const size_t off = (bytes + 255) & ~(size_t)255;
        bytes = off + b;
        return off;
    }
    // a matrix of parts {image offset, rows} in src_dt, stored as dst_dt
    void matrix(DevMatrix &M, int src_dt, int dst_dt, int K, std::initializer_list<std::pair<int64_t, int>> parts,
                bool f16_copy = false) {
        int Ntot = 0;
        for (auto &p : parts) Ntot += p.second;
        M.N = Ntot;
        M.K = K;
        M.fmt = wfmt(dst_dt);
        const size_t blocks = (size_t)(K / 32) * Ntot;
        if (dst_dt == DT_FP32) {
            fix.push_back({&M.q, take(blocks * 128)});
            if (pair_copies()) {
                fix.push_back({(const void **)&M.p16, take(blocks * 128)});
                fix.push_back({(const void **)&M.psc, take(blocks * 8)});
                pairs.push_back(&M);
            }
        } else {
            fix.push_back({&M.q, take(blocks * (block_bytes(dst_dt) - 4))});
            fix.push_back({(const void **)&M.sc, take(blocks * 4)});
            if (f16_copy) {
                fix.push_back({(const void **)&M.q16, take(blocks * 64)});
                expand.push_back(&M);
            }
        }
        int off = 0;
        for (auto &p : parts) {
            jobs.push_back({wfmt(src_dt), p.first, p.second, off, &M});
            off += p.second;
        }
    }
    // an FP32 vector concatenated from parts {image offset, floats}
    void vec(float *&v, std::initializer_list<std::pair<int64_t, int64_t>> parts) {
        int64_t n = 0;
        for (auto &p : parts) n += p.second;
        int64_t at = (int64_t)take((size_t)n * 4);
        fix.push_back({(const void **)&v, (size_t)at});
        for (auto &p : parts) {
            copies.push_back({p.first, at, p.second});
            at += 4 * p.second;
        }
    }
};

// Builds every device tensor of m from the image (a weights body in layout
// y on the device), storing the layer matrices as dst_dt.
int build_from_image(cih_model *m, const Layout &y, int dst_dt, const uint8_t *img) {
    const cih_config &c = m->cfg;
    const int64_t d = c.dim, F = c.hidden_dim, L = c.n_layers, V = c.vocab_size;
    Plan p;
    // token embedding: Q8_0 in Q8_0 models, FP32 otherwise (lib.rs:561, 675-687 vs 1113-1125)
    p.matrix(m->emb, y.emb_dtype, dst_dt == DT_Q8 ? DT_Q8 : DT_FP32, (int)d, {{y.emb, (int)V}});
    m->layers.resize(L);
    // The layer matrices of a quantized model also keep their quants as f16
    // integers (2 bytes per weight) for the LDS-staged GEMM of large batches;
    // CIH_GEMM_F16=0 leaves them out.
    const char *f16e = getenv("CIH_GEMM_F16");
    const bool f16 = dst_dt != DT_FP32 && !(f16e && !strcmp(f16e, "0"));
    for (int64_t l = 0; l < L; l++) {
        Layer &ly = m->layers[l];
        p.matrix(ly.wqkv, y.dtype, dst_dt, (int)d, {{y.wq[l], (int)d}, {y.wk[l], (int)d}, {y.wv[l], (int)d}}, f16);
        p.matrix(ly.wo, y.dtype, dst_dt, (int)d, {{y.wo[l], (int)d}}, f16);
        p.matrix(ly.w1, y.dtype, dst_dt, (int)d, {{y.fc1[l], (int)F}}, f16);
        p.matrix(ly.w2, y.dtype, dst_dt, (int)F, {{y.fc2[l], (int)d}}, f16);
        p.vec(ly.bqkv, {{y.bq[l], d}, {y.bk[l], d}, {y.bv[l], d}});
        p.vec(ly.bo, {{y.bo[l], d}});
        p.vec(ly.b1, {{y.fc1b[l], F}});
        p.vec(ly.b2, {{y.fc2b[l], d}});
        p.vec(ly.ln1w, {{y.ln1w[l], d}});
        p.vec(ly.ln1b, {{y.ln1b[l], d}});
        p.vec(ly.ln2w, {{y.ln2w[l], d}});
        p.vec(ly.ln2b, {{y.ln2b[l], d}});
    }
    p.vec(m->lnfw, {{y.lnfw, d}});
    p.vec(m->lnfb, {{y.lnfb, d}});
    // LM head (lib.rs:5379-5439), FP32 in every model
    m->has_head = y.head;
    if (y.head) {
        p.vec(m->lm_lnw, {{y.lm_lnw, d}});
        p.vec(m->lm_lnb, {{y.lm_lnb, d}});
        p.matrix(m->dense, DT_FP32, DT_FP32, (int)d, {{y.dense_w, (int)d}});
        p.vec(m->dense_b, {{y.dense_b, d}});
        p.matrix(m->dec, DT_FP32, DT_FP32, (int)d, {{y.dec_w, (int)V}});
        p.vec(m->dec_b, {{y.dec_b, V}});
    }

    uint8_t *arena = nullptr;
    HIPCHK(dalloc(arena, p.bytes, m->allocs));
    for (auto &f : p.fix) *f.first = arena + f.second;
    CopySeg *segs = nullptr;
    hipError_t e = hipMalloc(&segs, p.copies.size() * sizeof(CopySeg));
    if (e == hipSuccess)
        e = hipMemcpy(segs, p.copies.data(), p.copies.size() * sizeof(CopySeg), hipMemcpyHostToDevice);
    for (size_t i = 0; e == hipSuccess && i < p.jobs.size(); i++) {
        const Plan::Job &j = p.jobs[i];
        e = launch_load_matrix(img + j.src, j.src_fmt, j.N, *j.dst, j.n_off, m->stream);
    }
    for (size_t i = 0; e == hipSuccess && i < p.expand.size(); i++)
        e = launch_expand_f16(*p.expand[i], const_cast<unsigned short *>(p.expand[i]->q16), m->stream);
    for (size_t i = 0; e == hipSuccess && i < p.pairs.size(); i++)
        e = launch_pair_f16(*p.pairs[i], const_cast<unsigned short *>(p.pairs[i]->p16),
                            const_cast<float *>(p.pairs[i]->psc), m->stream);
    if (e == hipSuccess) e = launch_copy_segments(img, arena, segs, (int)p.copies.size(), m->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(m->stream);
    if (segs) hipFree(segs);
    if (e != hipSuccess) return set_error(CIH_ERR_HIP, "building the device model failed: %s", hipGetErrorString(e));
    m->dtype = dst_dt;
    return 0;
}

// Shared tail of both constructors: model shell, image, staging, GPU build,
// contact weights.
int create(const cih_config &cfg, const Layout &y, int dst_dt, int fd, const std::vector<Region> &regs,
           const float *contact_w, float contact_b, cih_model **out) {
    int dev_count = 0;
    if (hipGetDeviceCount(&dev_count) != hipSuccess || dev_count == 0)
        return set_error(CIH_ERR_HIP, "no HIP device available");
    cih_model *m = new cih_model();
    m->cfg = cfg;
    m->hd = cfg.dim / cfg.n_heads;
    const int64_t L = cfg.n_layers, H = cfg.n_heads;
    uint8_t *img = nullptr;
    auto fail = [&](int rc) {
        if (img) hipFree(img);
        cih_model_destroy(m);
        return rc;
    };
    if (hipGetDevice(&m->device) != hipSuccess || hipStreamCreate(&m->stream) != hipSuccess)
        return fail(set_error(CIH_ERR_HIP, "stream creation failed"));
    if (hipMalloc(&img, (size_t)y.total) != hipSuccess)
        return fail(set_error(CIH_ERR_HIP, "cannot allocate %lld bytes for the weights image", (long long)y.total));
    if (int rc = stage(m->device, fd, regs, img)) return fail(rc);
    if (int rc = build_from_image(m, y, dst_dt, img)) return fail(rc);
    hipFree(img);
    img = nullptr;

    // contact regression weights (EsmConfig::contact_head_weights, lib.rs:154-177)
    m->has_contacts = contact_w != nullptr;
    m->contact_b = contact_b;
    m->nz.assign(L, 0);
    if (m->has_contacts) {
        m->contact_w.assign(contact_w, contact_w + L * H);
        std::vector<int> heads(L * H, 0);
        for (int64_t l = 0; l < L; l++)
            for (int64_t h = 0; h < H; h++)
                if (m->contact_w[l * H + h] != 0.0f) heads[l * H + m->nz[l]++] = (int)h;
        int rc = upload(m, m->d_contact_w, m->contact_w.data(), m->contact_w.size());
        if (!rc) rc = upload(m, m->d_heads, heads.data(), heads.size());
        if (rc) return fail(rc);
    }
    *out = m;
    return CIH_OK;
}

}  // namespace

int upload_matrix(cih_model *m, int src_dt, int dst_dt, int K, const std::vector<Part> &parts, DevMatrix &out, bool pair) {
    if (src_dt != dst_dt && src_dt != DT_FP32) return set_error(CIH_ERR_ARG, "cannot convert dtype %d to %d", src_dt, dst_dt);
    int Ntot = 0;
    int64_t raw = 0;
    for (auto &p : parts) {
        Ntot += p.N;
        raw += mat_bytes(src_dt, (int64_t)p.N * K);
    }
    out.N = Ntot;
    out.K = K;
    out.fmt = wfmt(dst_dt);
    const size_t blocks = (size_t)(K / 32) * Ntot;
    if (dst_dt == DT_FP32) {
        float *q;
        HIPCHK(dalloc(q, blocks * 32, m->allocs));
        out.q = q;
        out.sc = nullptr;
    } else {
        uint8_t *q;
        float *sc;
        HIPCHK(dalloc(q, blocks * (block_bytes(dst_dt) - 4), m->allocs));
        HIPCHK(dalloc(sc, blocks, m->allocs));
        out.q = q;
        out.sc = sc;
    }
    uint8_t *img = nullptr;
    HIPCHK(hipMalloc(&img, (size_t)raw));
    hipError_t e = hipSuccess;
    int64_t at = 0;
    int n_off = 0;
    for (size_t i = 0; e == hipSuccess && i < parts.size(); i++) {
        const int64_t b = mat_bytes(src_dt, (int64_t)parts[i].N * K);
        e = hipMemcpy(img + at, parts[i].src, (size_t)b, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = launch_load_matrix(img + at, wfmt(src_dt), parts[i].N, out, n_off, nullptr);
        at += b;
        n_off += parts[i].N;
    }
    if (e == hipSuccess && dst_dt == DT_FP32 && pair && pair_copies()) {
        unsigned short *p16 = nullptr;
        float *psc = nullptr;
        e = dalloc(p16, blocks * 64, m->allocs);
        if (e == hipSuccess) e = dalloc(psc, blocks * 2, m->allocs);
        if (e == hipSuccess) {
            out.p16 = p16;
            out.psc = psc;
            e = launch_pair_f16(out, p16, psc, nullptr);
        }
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    hipFree(img);
    if (e != hipSuccess) return set_error(CIH_ERR_HIP, "matrix upload failed: %s", hipGetErrorString(e));
    return 0;
}

}  // namespace cih

using namespace cih;

extern "C" {

int cih_model_create(const cih_config *cfg, int32_t dtype, const cih_host_weights *w, const float *contact_w,
                     float contact_b, cih_model **out) {
    if (!out || !w) return set_error(CIH_ERR_ARG, "null argument");
    *out = nullptr;
    if (int rc = check_config(cfg)) return rc;
    if (dtype != DT_FP32 && dtype != DT_Q8 && dtype != DT_Q4) return set_error(CIH_ERR_ARG, "bad dtype %d", dtype);
    const void *need[] = {w->token_embedding_table, w->ln_1_weight, w->ln_1_bias, w->wq, w->bq, w->wk, w->bk, w->wv,
                          w->bv, w->wo, w->bo, w->ln_2_weight, w->ln_2_bias, w->fc1_weight, w->fc1_bias,
                          w->fc2_weight, w->fc2_bias, w->ln_f_weight, w->ln_f_bias};
    for (const void *p : need)
        if (!p) return set_error(CIH_ERR_ARG, "null weight tensor");
    const int64_t d = cfg->dim, F = cfg->hidden_dim, L = cfg->n_layers, V = cfg->vocab_size;
    // the caller's tensors laid out as one tensor-major body; the LM head is
    // used when the classifier holds all of it (lib.rs:5379-5439)
    const bool head = w->classifier_weights && w->classifier_len >= lm_head_floats(*cfg);
    const Layout y = grouped_layout(*cfg, dtype, head ? lm_head_floats(*cfg) : 0);
    std::vector<Region> regs;
    auto add = [&](const void *p, int64_t img_off, int64_t bytes) {
        regs.push_back({(const uint8_t *)p, 0, img_off, bytes});
    };
    add(w->token_embedding_table, y.emb, mat_bytes(y.emb_dtype, V * d));
    add(w->ln_1_weight, y.ln1w[0], 4 * L * d);
    add(w->ln_1_bias, y.ln1b[0], 4 * L * d);
    add(w->wq, y.wq[0], L * mat_bytes(dtype, d * d));
    add(w->bq, y.bq[0], 4 * L * d);
    add(w->wk, y.wk[0], L * mat_bytes(dtype, d * d));
    add(w->bk, y.bk[0], 4 * L * d);
    add(w->wv, y.wv[0], L * mat_bytes(dtype, d * d));
    add(w->bv, y.bv[0], 4 * L * d);
    add(w->wo, y.wo[0], L * mat_bytes(dtype, d * d));
    add(w->bo, y.bo[0], 4 * L * d);
    add(w->ln_2_weight, y.ln2w[0], 4 * L * d);
    add(w->ln_2_bias, y.ln2b[0], 4 * L * d);
    add(w->fc1_weight, y.fc1[0], L * mat_bytes(dtype, F * d));
    add(w->fc1_bias, y.fc1b[0], 4 * L * F);
    add(w->fc2_weight, y.fc2[0], L * mat_bytes(dtype, d * F));
    add(w->fc2_bias, y.fc2b[0], 4 * L * d);
    add(w->ln_f_weight, y.lnfw, 4 * d);
    add(w->ln_f_bias, y.lnfb, 4 * d);
    if (head) add(w->classifier_weights, y.lm_lnw, 4 * lm_head_floats(*cfg));
    return create(*cfg, y, dtype, -1, regs, contact_w, contact_b, out);
}

int cih_model_create_from_file(const char *path, int32_t quantize_to, const float *contact_w, float contact_b,
                               cih_model **out) {
    if (!path || !out) return set_error(CIH_ERR_ARG, "null argument");
    *out = nullptr;
    Fd f;
    f.fd = open(path, O_RDONLY);
    if (f.fd < 0) return set_error(CIH_ERR_IO, "cannot open %s", path);
    FileInfo fi;
    if (int rc = parse_file(path, f.fd, fi)) return rc;
    const int file_dt = fi.layout.dtype;
    int dst_dt = file_dt;
    if (quantize_to == DT_Q8 || quantize_to == DT_Q4) {
        if (file_dt != DT_FP32 && file_dt != quantize_to)
            return set_error(CIH_ERR_ARG, "cannot requantize a dtype %d file to %d", file_dt, quantize_to);
        dst_dt = quantize_to;
    } else if (quantize_to != -1 && quantize_to != file_dt) {
        return set_error(CIH_ERR_ARG, "bad quantize_to %d", quantize_to);
    }
    if (int rc = check_config(&fi.cfg)) return rc;
#ifdef POSIX_FADV_SEQUENTIAL
    posix_fadvise(f.fd, 0, 0, POSIX_FADV_SEQUENTIAL);
#endif
    return create(fi.cfg, fi.layout, dst_dt, f.fd, {{nullptr, fi.body_off, 0, fi.layout.total}}, contact_w, contact_b,
                  out);
}

}  // extern "C"
