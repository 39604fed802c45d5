// llm_accel.cpp -- C ABI of the resident decoder-layer path (host side).
//
// One context owns every device allocation: weights in the tile4x128
// layout, the norm table, the Q8.8 RoPE table, the paged KV cache, hidden
// pairs and scratch.  llm_task() validates a command in the controller's
// order, enqueues the sublayer's kernels on the context stream and returns
// the status record; nothing of the hidden state or KV cache crosses PCIe
// between tasks.
#include "llm_accel.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "kernels.h"

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

#define HIP_TRY(expr)                                                   \
    do {                                                                \
        hipError_t e_ = (expr);                                         \
        if (e_ != hipSuccess)                                           \
            return fail(LLM_E_HIP, std::string(#expr) + ": " +          \
                                       hipGetErrorString(e_));          \
    } while (0)

uint32_t round_up(uint32_t v, uint32_t m) { return (v + m - 1) / m * m; }
uint64_t cdiv(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

// One weight matrix in the tile4x128 layout.
struct Matrix {
    int16_t* d = nullptr;
    uint32_t n = 0, k = 0, n_pad = 0, k_pad = 0, steps = 0;
    int maxw[3] = {0, 0, 0};  // per stored projection (qkv keeps three)
    int L = 16;               // int32 widening interval in k-steps
    size_t elems() const { return (size_t)n_pad * k_pad; }
};

enum { M_QKV = 0, M_O = 1, M_GATE = 2, M_UP = 3, M_DOWN = 4, M_COUNT = 5 };

// Largest int32 accumulation interval (k-steps of 8 products per lane)
// that cannot overflow for any int16 activation: 8 * L * 32768 * max|w|
// < 2^31.  0 selects the per-product int64 path.
int widening_interval(int maxw) {
    if (maxw == 0) return 16;
    const int64_t lim = ((int64_t)1 << 31) - 1;
    const int64_t per_step = (int64_t)8 * 32768 * maxw;
    const int64_t allowed = lim / per_step;
    for (int L : {16, 8, 4, 1})
        if (allowed >= L) return L;
    return 0;
}

}  // namespace

struct llm_ctx {
    llm_shape_t s{};
    int device = 0;
    hipStream_t stream = nullptr;
    uint32_t H = 0, I = 0, Hq = 0, Hkv = 0, d = 0, G = 0, Ckv = 0, L = 0;
    uint32_t max_seq = 0, tiles = 0, Hp = 0, Ip = 0, Nqkv = 0;
    int32_t qk_scale = 0;
    int16_t* arena = nullptr;          // all weights
    std::vector<Matrix> mats;          // [layer][M_COUNT]
    std::vector<bool> loaded;          // [layer][7]
    bool norms_loaded = false;
    int16_t* norms = nullptr;
    int16_t* rope = nullptr;
    int16_t* exp8 = nullptr;
    int16_t* exp14 = nullptr;
    int16_t* kcache = nullptr;
    int16_t* vcache = nullptr;
    int32_t* page_table = nullptr;     // [layer][kv_head][tile]
    std::vector<int32_t> host_pages;
    std::vector<int16_t*> pairs;       // [8][Hp]
    int16_t* xn = nullptr;             // [8][Hp]
    int16_t* qkv = nullptr;            // [8][Nqkv]
    int16_t* q = nullptr;              // [8][H]
    int16_t* attn = nullptr;           // [8][Hp]
    int16_t* act = nullptr;            // [8][Ip]
    std::vector<void*> allocations;
    std::vector<hipEvent_t> events;

    Matrix& mat(uint32_t layer, int m) { return mats[layer * M_COUNT + m]; }
};

namespace {

int dev_alloc(llm_ctx* c, void** p, size_t bytes) {
    hipError_t e = hipMalloc(p, bytes);
    if (e != hipSuccess)
        return fail(LLM_E_NOMEM, "hipMalloc(" + std::to_string(bytes) +
                                     "): " + hipGetErrorString(e));
    c->allocations.push_back(*p);
    e = hipMemset(*p, 0, bytes);
    if (e != hipSuccess) return fail(LLM_E_HIP, hipGetErrorString(e));
    return 0;
}

// exp tables: floor(e^x * 2^F) for x = -2048/256 .. 0.
void build_exp_tables(int16_t* q8_8, int16_t* q2_14) {
    for (int x = -2048; x <= 0; x++) {
        long double e = expl((long double)x / 256.0L);
        q8_8[x + 2048] = (int16_t)floorl(e * 256.0L);
        q2_14[x + 2048] = (int16_t)floorl(e * 16384.0L);
    }
}

int16_t quantize_fix16(double v) {  // host/host_qwen_8x64.cpp:496-505
    double s = std::round(v * 256.0);
    if (s > 32767.0) return 32767;
    if (s < -32768.0) return -32768;
    return (int16_t)s;
}

// Rows [row0, row0 + rows) of matrix m get row-major weights w[rows][k].
int upload_rows(llm_ctx* c, Matrix& m, uint32_t row0, uint32_t rows,
                const int16_t* w, int which) {
    if (row0 % llm::kBlockRows != 0)
        return fail(LLM_E_ARG, "projection rows not aligned to 4");
    const uint32_t rows_pad = round_up(rows, llm::kBlockRows);
    const uint32_t S = m.steps;
    std::vector<int16_t> buf((size_t)rows_pad * m.k_pad, 0);
    int maxw = 0;
    for (uint32_t n = 0; n < rows; n++) {
        const uint32_t b = n / 4, i = n % 4;
        const int16_t* src = w + (size_t)n * m.k;
        for (uint32_t k = 0; k < m.k; k++) {
            const uint32_t s = k / 128, j = (k % 128) / 8, e = k % 8;
            const int16_t v = src[k];
            buf[(((size_t)b * S + s) * 4 + i) * 128 + j * 8 + e] = v;
            maxw = std::max(maxw, std::abs((int)v));
        }
    }
    const size_t off = (size_t)(row0 / 4) * S * 512;
    HIP_TRY(hipMemcpy(m.d + off, buf.data(), buf.size() * sizeof(int16_t),
                      hipMemcpyHostToDevice));
    m.maxw[which] = maxw;
    m.L = widening_interval(std::max({m.maxw[0], m.maxw[1], m.maxw[2]}));
    return 0;
}

// Controller schedule counters for one accepted command
// (kernel/control_cache_8x64.cpp:5974-6481, attention tasks :5764,
// vector tasks :1856-1929).
void fill_counters(const llm_ctx* c, uint32_t op, uint32_t R, uint32_t pos,
                   llm_status_t* st) {
    const uint32_t vt = (R > 0 ? 1u : 0u) + (R > 4 ? 1u : 0u);
    const uint32_t hp = R * (uint32_t)cdiv(c->H, 16);
    const uint32_t ip = R * (uint32_t)cdiv(c->I, 16);
    if (op == LLM_OP_FINAL_NORM) {
        st->vector_tasks = vt;
        st->completed_packets = hp;
        return;
    }
    uint32_t waves = 0, mm = 0, vec = vt, pk = hp;
    const uint32_t begin = op == LLM_OP_FFN_SUBLAYER ? 4 : 0;
    const uint32_t end = op == LLM_OP_ATTENTION_SUBLAYER ? 4 : 7;
    for (uint32_t step = begin; step < end; step++) {
        const uint32_t out_dim = (step == 1 || step == 2) ? c->Ckv
                               : (step == 4 || step == 5) ? c->I : c->H;
        if (step == 3) {
            const uint32_t ow = (uint32_t)cdiv(c->d, 64);
            uint32_t at = 0;
            for (uint32_t t = 0; t < R; t++)
                at += 2 * (uint32_t)cdiv(pos + t + 1, 64) * (1 + ow);
            mm += at;
            pk += at * 32;
            waves += at / 2;
        }
        const uint32_t w = (uint32_t)cdiv(out_dim, 128);
        waves += w;
        mm += 2 * w;
        pk += 2 * w * 32;
        if (step == 3) {
            vec += vt;
            pk += hp;
            if (op != LLM_OP_ATTENTION_SUBLAYER) {
                vec += vt;
                pk += hp;
            }
        } else if (step == 5) {
            vec += vt;
            pk += ip;
        } else if (step == 6) {
            vec += vt;
            pk += hp;
        }
    }
    st->output_waves = waves;
    st->mm_tasks = mm;
    st->vector_tasks = vec;
    st->completed_packets = pk;
}

int check_layer_loaded(llm_ctx* c, uint32_t layer, bool attn, bool ffn) {
    if (!c->norms_loaded) return fail(LLM_E_STATE, "norm table not loaded");
    for (uint32_t p = 0; p < 7; p++) {
        const bool need = p < 4 ? attn : ffn;
        if (need && !c->loaded[layer * 7 + p])
            return fail(LLM_E_STATE, "layer " + std::to_string(layer) +
                                         " projection " + std::to_string(p) +
                                         " not loaded");
    }
    return 0;
}

int enqueue_attention_sublayer(llm_ctx* c, uint32_t layer, uint32_t R,
                               uint32_t pos, const int16_t* in, int16_t* out) {
    hipStream_t st = c->stream;
    HIP_TRY(llm::launch_rmsnorm(in, c->Hp, c->norms + (size_t)(2 * layer) * c->H,
                                c->H, c->xn, c->Hp, R, st));
    const Matrix& mq = c->mat(layer, M_QKV);
    llm::ProjArgs a{};
    a.w0 = mq.d;
    a.steps = mq.steps;
    a.x = c->xn;
    a.ldx = c->Hp;
    a.out = c->qkv;
    a.ldo = c->Nqkv;
    a.n = mq.n;
    a.rows = R;
    HIP_TRY(llm::launch_proj(a, llm::EPI_STORE, mq.L, mq.n_pad / 4, st));
    const int32_t* pt = c->page_table + (size_t)layer * c->Hkv * c->tiles;
    llm::RopeArgs r{};
    r.qkv = c->qkv;
    r.ldqkv = c->Nqkv;
    r.q = c->q;
    r.ldq = c->H;
    r.kcache = c->kcache;
    r.vcache = c->vcache;
    r.page_table = pt;
    r.tiles = c->tiles;
    r.rope = c->rope;
    r.pos0 = pos;
    r.num_heads = c->Hq;
    r.num_kv_heads = c->Hkv;
    r.head_dim = c->d;
    HIP_TRY(llm::launch_rope_append(r, R, st));
    llm::AttnArgs at{};
    at.q = c->q;
    at.ldq = c->H;
    at.kcache = c->kcache;
    at.vcache = c->vcache;
    at.page_table = pt;
    at.tiles = c->tiles;
    at.pos0 = pos;
    at.group = c->G;
    at.head_dim = c->d;
    at.qk_scale = c->qk_scale;
    at.exp14 = c->exp14;
    at.out = c->attn;
    at.ldo = c->Hp;
    HIP_TRY(llm::launch_attention(at, R, c->Hkv, st));
    const Matrix& mo = c->mat(layer, M_O);
    llm::ProjArgs o{};
    o.w0 = mo.d;
    o.steps = mo.steps;
    o.x = c->attn;
    o.ldx = c->Hp;
    o.out = out;
    o.ldo = c->Hp;
    o.res = in;
    o.ldr = c->Hp;
    o.n = mo.n;
    o.rows = R;
    HIP_TRY(llm::launch_proj(o, llm::EPI_RESID, mo.L, mo.n_pad / 4, st));
    return 0;
}

int enqueue_ffn_sublayer(llm_ctx* c, uint32_t layer, uint32_t R,
                         const int16_t* in, int16_t* out) {
    hipStream_t st = c->stream;
    HIP_TRY(llm::launch_rmsnorm(in, c->Hp,
                                c->norms + (size_t)(2 * layer + 1) * c->H,
                                c->H, c->xn, c->Hp, R, st));
    const Matrix& mg = c->mat(layer, M_GATE);
    const Matrix& mu = c->mat(layer, M_UP);
    llm::ProjArgs a{};
    a.w0 = mg.d;
    a.w1 = mu.d;
    a.steps = mg.steps;
    a.x = c->xn;
    a.ldx = c->Hp;
    a.out = c->act;
    a.ldo = c->Ip;
    a.n = mg.n;
    a.rows = R;
    a.exp8 = c->exp8;
    HIP_TRY(llm::launch_proj(a, llm::EPI_SILU, std::min(mg.L, mu.L) == 0 ? 0 :
                             std::min(mg.L, mu.L), mg.n_pad / 4, st));
    const Matrix& md = c->mat(layer, M_DOWN);
    llm::ProjArgs dn{};
    dn.w0 = md.d;
    dn.steps = md.steps;
    dn.x = c->act;
    dn.ldx = c->Ip;
    dn.out = out;
    dn.ldo = c->Hp;
    dn.res = in;
    dn.ldr = c->Hp;
    dn.n = md.n;
    dn.rows = R;
    HIP_TRY(llm::launch_proj(dn, llm::EPI_RESID, md.L, md.n_pad / 4, st));
    return 0;
}

}  // namespace

extern "C" {

const char* llm_last_error(void) { return g_err.c_str(); }

int llm_ctx_create(const llm_shape_t* shape, int device, uint32_t num_pairs,
                   llm_ctx_t** out) {
    if (!shape || !out) return fail(LLM_E_ARG, "null argument");
    *out = nullptr;
    const llm_shape_t& s = *shape;
    if (s.hidden_size == 0 || s.intermediate_size == 0 || s.num_layers == 0 ||
        s.num_heads == 0 || s.num_kv_heads == 0 || s.max_seq_len == 0 ||
        s.hidden_size % s.num_heads != 0 || s.num_heads % s.num_kv_heads != 0)
        return fail(LLM_E_ARG, "inconsistent shape");
    const uint32_t d = s.hidden_size / s.num_heads;
    const uint32_t G = s.num_heads / s.num_kv_heads;
    if (d % 2 != 0 || d > 128 || G > 16 || G * d > 2048)
        return fail(LLM_E_ARG, "head_dim must be even and <= 128, group <= 16");
    if (s.hidden_size % 4 || s.intermediate_size % 4 || (s.num_kv_heads * d) % 4)
        return fail(LLM_E_ARG, "hidden, intermediate and KV widths must be multiples of 4");
    if (num_pairs < 2) return fail(LLM_E_ARG, "need at least two hidden pairs");
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0)
        return fail(LLM_E_HIP, "no HIP device available");
    if (device < 0 || device >= ndev) return fail(LLM_E_ARG, "bad device id");
    HIP_TRY(hipSetDevice(device));

    llm_ctx* c = new llm_ctx();
    c->s = s;
    c->device = device;
    c->H = s.hidden_size;
    c->I = s.intermediate_size;
    c->Hq = s.num_heads;
    c->Hkv = s.num_kv_heads;
    c->d = d;
    c->G = G;
    c->Ckv = s.num_kv_heads * d;
    c->L = s.num_layers;
    c->max_seq = s.max_seq_len;
    c->tiles = (uint32_t)cdiv(s.max_seq_len, llm::kTile);
    c->Hp = round_up(c->H, llm::kStepCols);
    c->Ip = round_up(c->I, llm::kStepCols);
    c->Nqkv = c->H + 2 * c->Ckv;
    c->qk_scale = (int32_t)std::floor(256.0 / std::sqrt((double)d) + 0.5);

    auto cleanup = [&](int code) {
        llm_ctx_destroy(c);
        return code;
    };
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess)
        return cleanup(fail(LLM_E_HIP, "hipStreamCreate failed"));

    // weights
    c->mats.resize((size_t)c->L * M_COUNT);
    c->loaded.assign((size_t)c->L * 7, false);
    size_t total = 0;
    for (uint32_t l = 0; l < c->L; l++) {
        const uint32_t dims[M_COUNT][2] = {{c->Nqkv, c->H}, {c->H, c->H},
                                           {c->I, c->H}, {c->I, c->H},
                                           {c->H, c->I}};
        for (int m = 0; m < M_COUNT; m++) {
            Matrix& mt = c->mat(l, m);
            mt.n = dims[m][0];
            mt.k = dims[m][1];
            mt.n_pad = round_up(mt.n, llm::kBlockRows);
            mt.k_pad = round_up(mt.k, llm::kStepCols);
            mt.steps = mt.k_pad / llm::kStepCols;
            total += mt.elems();
        }
    }
    int rc;
    if ((rc = dev_alloc(c, (void**)&c->arena, total * sizeof(int16_t))))
        return cleanup(rc);
    size_t off = 0;
    for (auto& mt : c->mats) {
        mt.d = c->arena + off;
        off += mt.elems();
    }
    // tables
    if ((rc = dev_alloc(c, (void**)&c->norms,
                        (size_t)(2 * c->L + 1) * c->H * sizeof(int16_t))) ||
        (rc = dev_alloc(c, (void**)&c->rope,
                        (size_t)c->max_seq * d * sizeof(int16_t))) ||
        (rc = dev_alloc(c, (void**)&c->exp8, 2049 * sizeof(int16_t))) ||
        (rc = dev_alloc(c, (void**)&c->exp14, 2049 * sizeof(int16_t))))
        return cleanup(rc);
    {
        // aux1 RoPE table exactly as initialize_persistent_auxiliary_data
        // (host/host_qwen_8x64.cpp:2159-2189): [cos d/2 | sin d/2] per pos.
        std::vector<int16_t> rope((size_t)c->max_seq * d);
        std::vector<double> inv_freq(d / 2);
        for (uint32_t i = 0; i < d / 2; i++)
            inv_freq[i] = 1.0 / std::pow(s.rope_theta, double(2 * i) / d);
        for (uint32_t p = 0; p < c->max_seq; p++)
            for (uint32_t i = 0; i < d / 2; i++) {
                const double angle = p * inv_freq[i];
                rope[(size_t)p * d + i] = quantize_fix16(std::cos(angle));
                rope[(size_t)p * d + d / 2 + i] = quantize_fix16(std::sin(angle));
            }
        if (hipMemcpy(c->rope, rope.data(), rope.size() * 2, hipMemcpyHostToDevice))
            return cleanup(fail(LLM_E_HIP, "rope upload"));
        int16_t e8[2049], e14[2049];
        build_exp_tables(e8, e14);
        if (hipMemcpy(c->exp8, e8, sizeof(e8), hipMemcpyHostToDevice) ||
            hipMemcpy(c->exp14, e14, sizeof(e14), hipMemcpyHostToDevice))
            return cleanup(fail(LLM_E_HIP, "exp table upload"));
    }
    // paged KV cache: pages of 64 positions per (layer, kv head); the
    // default page table maps tile t of (layer, head) to page
    // (layer * Hkv + head) * tiles + t.
    const size_t pages = (size_t)c->L * c->Hkv * c->tiles;
    if ((rc = dev_alloc(c, (void**)&c->kcache, pages * llm::kTile * d * 2)) ||
        (rc = dev_alloc(c, (void**)&c->vcache, pages * llm::kTile * d * 2)) ||
        (rc = dev_alloc(c, (void**)&c->page_table, pages * sizeof(int32_t))))
        return cleanup(rc);
    c->host_pages.resize(pages);
    for (size_t i = 0; i < pages; i++) c->host_pages[i] = (int32_t)i;
    if (hipMemcpy(c->page_table, c->host_pages.data(), pages * 4,
                  hipMemcpyHostToDevice))
        return cleanup(fail(LLM_E_HIP, "page table upload"));
    // hidden pairs and scratch
    c->pairs.resize(num_pairs);
    for (auto& p : c->pairs)
        if ((rc = dev_alloc(c, (void**)&p, (size_t)8 * c->Hp * 2)))
            return cleanup(rc);
    if ((rc = dev_alloc(c, (void**)&c->xn, (size_t)8 * c->Hp * 2)) ||
        (rc = dev_alloc(c, (void**)&c->qkv, (size_t)8 * c->Nqkv * 2)) ||
        (rc = dev_alloc(c, (void**)&c->q, (size_t)8 * c->H * 2)) ||
        (rc = dev_alloc(c, (void**)&c->attn, (size_t)8 * c->Hp * 2)) ||
        (rc = dev_alloc(c, (void**)&c->act, (size_t)8 * c->Ip * 2)))
        return cleanup(rc);
    *out = c;
    return 0;
}

void llm_ctx_destroy(llm_ctx_t* c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    for (auto e : c->events) (void)hipEventDestroy(e);
    for (void* p : c->allocations) (void)hipFree(p);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
}

int llm_load_projection(llm_ctx_t* c, uint32_t layer, uint32_t proj,
                        const int16_t* w) {
    if (!c || !w || layer >= c->L || proj > LLM_PROJ_DOWN)
        return fail(LLM_E_ARG, "bad projection load arguments");
    HIP_TRY(hipSetDevice(c->device));
    int rc;
    switch (proj) {
    case LLM_PROJ_Q:
        rc = upload_rows(c, c->mat(layer, M_QKV), 0, c->H, w, 0);
        break;
    case LLM_PROJ_K:
        rc = upload_rows(c, c->mat(layer, M_QKV), c->H, c->Ckv, w, 1);
        break;
    case LLM_PROJ_V:
        rc = upload_rows(c, c->mat(layer, M_QKV), c->H + c->Ckv, c->Ckv, w, 2);
        break;
    case LLM_PROJ_O:
        rc = upload_rows(c, c->mat(layer, M_O), 0, c->H, w, 0);
        break;
    case LLM_PROJ_GATE:
        rc = upload_rows(c, c->mat(layer, M_GATE), 0, c->I, w, 0);
        break;
    case LLM_PROJ_UP:
        rc = upload_rows(c, c->mat(layer, M_UP), 0, c->I, w, 0);
        break;
    default:
        rc = upload_rows(c, c->mat(layer, M_DOWN), 0, c->H, w, 0);
        break;
    }
    if (rc == 0) c->loaded[layer * 7 + proj] = true;
    return rc;
}

int llm_load_packed_shards(llm_ctx_t* c, const int16_t* const shards[16],
                           uint64_t shard_words) {
    if (!c || !shards) return fail(LLM_E_ARG, "null argument");
    for (int i = 0; i < 16; i++)
        if (!shards[i]) return fail(LLM_E_ARG, "null shard");
    // projection_spec / projection_weight_raw (host:325-376, :899-935)
    uint64_t tiles[7], base[7], layer_tiles = 0;
    uint32_t in_dims[7], out_dims[7];
    for (uint32_t p = 0; p < 7; p++) {
        in_dims[p] = p == LLM_PROJ_DOWN ? c->I : c->H;
        out_dims[p] = (p == LLM_PROJ_K || p == LLM_PROJ_V) ? c->Ckv
                    : (p == LLM_PROJ_GATE || p == LLM_PROJ_UP) ? c->I : c->H;
        tiles[p] = cdiv(out_dims[p], 16) * cdiv(in_dims[p], 16);
        base[p] = layer_tiles;
        layer_tiles += tiles[p];
    }
    if (shard_words < cdiv((uint64_t)c->L * layer_tiles, 2))
        return fail(LLM_E_ARG, "shard_words too small for the shape");
    std::vector<int16_t> w;
    for (uint32_t l = 0; l < c->L; l++) {
        for (uint32_t p = 0; p < 7; p++) {
            const uint32_t N = out_dims[p], K = in_dims[p];
            const uint64_t in_tiles = cdiv(K, 16);
            w.assign((size_t)N * K, 0);
            for (uint32_t n = 0; n < N; n++)
                for (uint32_t k = 0; k < K; k++) {
                    const uint64_t tile = (uint64_t)l * layer_tiles + base[p] +
                                          (uint64_t)(n / 16) * in_tiles + k / 16;
                    const uint32_t lane_in_tile = (n % 16) * 16 + k % 16;
                    const uint32_t shard = (uint32_t)(tile & 1) * 8 + lane_in_tile / 32;
                    w[(size_t)n * K + k] =
                        shards[shard][(tile >> 1) * 32 + lane_in_tile % 32];
                }
            int rc = llm_load_projection(c, l, p, w.data());
            if (rc) return rc;
        }
    }
    return 0;
}

int llm_load_norms(llm_ctx_t* c, const int16_t* norms) {
    if (!c || !norms) return fail(LLM_E_ARG, "null argument");
    HIP_TRY(hipSetDevice(c->device));
    HIP_TRY(hipMemcpy(c->norms, norms, (size_t)(2 * c->L + 1) * c->H * 2,
                      hipMemcpyHostToDevice));
    c->norms_loaded = true;
    return 0;
}

int llm_hidden_upload(llm_ctx_t* c, uint32_t pair, const int16_t* rows,
                      uint32_t n) {
    if (!c || !rows || pair >= c->pairs.size() || n > 8)
        return fail(LLM_E_ARG, "bad hidden upload arguments");
    HIP_TRY(hipSetDevice(c->device));
    HIP_TRY(hipMemcpy2DAsync(c->pairs[pair], (size_t)c->Hp * 2, rows,
                             (size_t)c->H * 2, (size_t)c->H * 2, n,
                             hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return 0;
}

int llm_hidden_download(llm_ctx_t* c, uint32_t pair, int16_t* rows,
                        uint32_t n) {
    if (!c || !rows || pair >= c->pairs.size() || n > 8)
        return fail(LLM_E_ARG, "bad hidden download arguments");
    HIP_TRY(hipSetDevice(c->device));
    HIP_TRY(hipMemcpy2DAsync(rows, (size_t)c->H * 2, c->pairs[pair],
                             (size_t)c->Hp * 2, (size_t)c->H * 2, n,
                             hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return 0;
}

int llm_hidden_upload_ports(llm_ctx_t* c, uint32_t pair, const int16_t* port0,
                            const int16_t* port1, uint32_t n,
                            uint32_t stride_words) {
    if (!c || !port0 || (n > 4 && !port1) || n > 8 ||
        (size_t)stride_words * 32 < c->H)
        return fail(LLM_E_ARG, "bad port upload arguments");
    std::vector<int16_t> rows((size_t)n * c->H);
    for (uint32_t t = 0; t < n; t++) {
        const int16_t* src = (t < 4 ? port0 : port1) + (size_t)(t % 4) * stride_words * 32;
        std::memcpy(&rows[(size_t)t * c->H], src, (size_t)c->H * 2);
    }
    return llm_hidden_upload(c, pair, rows.data(), n);
}

int llm_hidden_download_ports(llm_ctx_t* c, uint32_t pair, int16_t* port0,
                              int16_t* port1, uint32_t n,
                              uint32_t stride_words) {
    if (!c || !port0 || (n > 4 && !port1) || n > 8 ||
        (size_t)stride_words * 32 < c->H)
        return fail(LLM_E_ARG, "bad port download arguments");
    std::vector<int16_t> rows((size_t)n * c->H);
    int rc = llm_hidden_download(c, pair, rows.data(), n);
    if (rc) return rc;
    for (uint32_t t = 0; t < n; t++) {
        int16_t* dst = (t < 4 ? port0 : port1) + (size_t)(t % 4) * stride_words * 32;
        std::memcpy(dst, &rows[(size_t)t * c->H], (size_t)c->H * 2);
    }
    return 0;
}

int llm_task(llm_ctx_t* c, uint32_t op, uint32_t layer, uint32_t token_count,
             uint32_t position, uint32_t tile_len, uint32_t in_pair,
             uint32_t out_pair, llm_status_t* status) {
    llm_status_t local;
    llm_status_t* st = status ? status : &local;
    std::memset(st, 0, sizeof(*st));
    if (!c) return fail(LLM_E_ARG, "null context");
    if (in_pair >= c->pairs.size() || out_pair >= c->pairs.size())
        return fail(LLM_E_ARG, "bad pair id");
    // control_cache_8x64_dual_core (kernel/control_cache_8x64.cpp:5882-5957)
    if (tile_len != 0) token_count &= 0xffffu;
    st->op = LLM_OP_NOP;
    st->token_count = token_count;
    st->last_task = 1;
    auto reject = [&](uint32_t code) {
        st->code = code;
        return (int)code;
    };
    if (token_count > 8) return reject(LLM_STATUS_BAD_TOKEN_COUNT);
    st->op = op;
    if (op > LLM_OP_FINAL_NORM) return reject(LLM_STATUS_BAD_OPERATOR);
    if (op == LLM_OP_NOP) return LLM_STATUS_OK;
    if (layer >= c->L) return reject(LLM_STATUS_BAD_LAYER);
    const int16_t* in = c->pairs[in_pair];
    int16_t* out = c->pairs[out_pair];
    if (hipSetDevice(c->device) != hipSuccess)
        return fail(LLM_E_HIP, "hipSetDevice failed");
    if (op == LLM_OP_FINAL_NORM) {
        if (token_count == 0) return reject(LLM_STATUS_BAD_TOKEN_COUNT);
        if (!c->norms_loaded) return fail(LLM_E_STATE, "norm table not loaded");
        HIP_TRY(llm::launch_rmsnorm(in, c->Hp,
                                    c->norms + (size_t)(2 * c->L) * c->H, c->H,
                                    out, c->Hp, token_count, c->stream));
        fill_counters(c, op, token_count, position, st);
        return LLM_STATUS_OK;
    }
    if (op == LLM_OP_DECODER_LAYER || op == LLM_OP_ATTENTION_SUBLAYER ||
        op == LLM_OP_FFN_SUBLAYER) {
        if (token_count == 0) return reject(LLM_STATUS_BAD_TOKEN_COUNT);
        if (position >= c->max_seq || position + token_count > c->max_seq)
            return reject(LLM_STATUS_BAD_POSITION);
        int rc = check_layer_loaded(c, layer, op != LLM_OP_FFN_SUBLAYER,
                                    op != LLM_OP_ATTENTION_SUBLAYER);
        if (rc) return rc;
        if (op == LLM_OP_ATTENTION_SUBLAYER) {
            rc = enqueue_attention_sublayer(c, layer, token_count, position, in, out);
        } else if (op == LLM_OP_FFN_SUBLAYER) {
            rc = enqueue_ffn_sublayer(c, layer, token_count, in, out);
        } else {
            rc = enqueue_attention_sublayer(c, layer, token_count, position, in, out);
            if (rc == 0) rc = enqueue_ffn_sublayer(c, layer, token_count, out, out);
        }
        if (rc) return rc;
        fill_counters(c, op, token_count, position, st);
        return LLM_STATUS_OK;
    }
    // The resident-layer image carries no per-operator scheduler
    // (kernel/control_cache_8x64.cpp:6483-6494).
    return reject(LLM_STATUS_BAD_OPERATOR);
}

int llm_kv_read(llm_ctx_t* c, uint32_t layer, uint32_t h, uint32_t pos0,
                uint32_t n, int16_t* k, int16_t* v) {
    if (!c || layer >= c->L || h >= c->Hkv || pos0 + n > c->max_seq)
        return fail(LLM_E_ARG, "bad KV read arguments");
    HIP_TRY(hipSetDevice(c->device));
    HIP_TRY(hipStreamSynchronize(c->stream));
    for (uint32_t p = pos0; p < pos0 + n;) {
        const uint32_t tile = p / 64, slot = p % 64;
        const uint32_t cnt = std::min(64 - slot, pos0 + n - p);
        const size_t page = c->host_pages[((size_t)layer * c->Hkv + h) * c->tiles + tile];
        const size_t off = (page * 64 + slot) * c->d;
        if (k) HIP_TRY(hipMemcpy(k + (size_t)(p - pos0) * c->d, c->kcache + off,
                                 (size_t)cnt * c->d * 2, hipMemcpyDeviceToHost));
        if (v) HIP_TRY(hipMemcpy(v + (size_t)(p - pos0) * c->d, c->vcache + off,
                                 (size_t)cnt * c->d * 2, hipMemcpyDeviceToHost));
        p += cnt;
    }
    return 0;
}

int llm_kv_write(llm_ctx_t* c, uint32_t layer, uint32_t h, uint32_t pos0,
                 uint32_t n, const int16_t* k, const int16_t* v) {
    if (!c || layer >= c->L || h >= c->Hkv || pos0 + n > c->max_seq)
        return fail(LLM_E_ARG, "bad KV write arguments");
    HIP_TRY(hipSetDevice(c->device));
    HIP_TRY(hipStreamSynchronize(c->stream));
    for (uint32_t p = pos0; p < pos0 + n;) {
        const uint32_t tile = p / 64, slot = p % 64;
        const uint32_t cnt = std::min(64 - slot, pos0 + n - p);
        const size_t page = c->host_pages[((size_t)layer * c->Hkv + h) * c->tiles + tile];
        const size_t off = (page * 64 + slot) * c->d;
        if (k) HIP_TRY(hipMemcpy(c->kcache + off, k + (size_t)(p - pos0) * c->d,
                                 (size_t)cnt * c->d * 2, hipMemcpyHostToDevice));
        if (v) HIP_TRY(hipMemcpy(c->vcache + off, v + (size_t)(p - pos0) * c->d,
                                 (size_t)cnt * c->d * 2, hipMemcpyHostToDevice));
        p += cnt;
    }
    return 0;
}

int llm_kv_clear(llm_ctx_t* c) {
    if (!c) return fail(LLM_E_ARG, "null context");
    HIP_TRY(hipSetDevice(c->device));
    const size_t bytes = (size_t)c->L * c->Hkv * c->tiles * 64 * c->d * 2;
    HIP_TRY(hipMemsetAsync(c->kcache, 0, bytes, c->stream));
    HIP_TRY(hipMemsetAsync(c->vcache, 0, bytes, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return 0;
}

void* llm_pair_device_ptr(llm_ctx_t* c, uint32_t pair) {
    return (c && pair < c->pairs.size()) ? c->pairs[pair] : nullptr;
}

void* llm_stream(llm_ctx_t* c) { return c ? (void*)c->stream : nullptr; }

int llm_sync(llm_ctx_t* c) {
    if (!c) return fail(LLM_E_ARG, "null context");
    HIP_TRY(hipSetDevice(c->device));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return 0;
}

int llm_event_record(llm_ctx_t* c, uint32_t slot) {
    if (!c || slot >= 64) return fail(LLM_E_ARG, "bad event slot");
    HIP_TRY(hipSetDevice(c->device));
    if (c->events.empty()) {
        c->events.resize(64);
        for (auto& e : c->events) HIP_TRY(hipEventCreate(&e));
    }
    HIP_TRY(hipEventRecord(c->events[slot], c->stream));
    return 0;
}

int llm_event_elapsed_ms(llm_ctx_t* c, uint32_t a, uint32_t b, float* ms) {
    if (!c || !ms || a >= c->events.size() || b >= c->events.size())
        return fail(LLM_E_ARG, "bad event slots");
    HIP_TRY(hipEventSynchronize(c->events[b]));
    HIP_TRY(hipEventElapsedTime(ms, c->events[a], c->events[b]));
    return 0;
}

int llm_exp_tables(int16_t* q8_8, int16_t* q2_14) {
    int16_t a[2049], b[2049];
    build_exp_tables(a, b);
    if (q8_8) std::memcpy(q8_8, a, sizeof(a));
    if (q2_14) std::memcpy(q2_14, b, sizeof(b));
    return 0;
}

}  // extern "C"
