// kmamba_model.hip - the stacked model of the reference (token embedding,
// n_layers Mamba-3 blocks, output head) behind its C API: create / free /
// init, checkpoint version 4 save / load, and the forward on the GPU.
//
// Forward (ref src/kmamba.c:344-372): the embedding rows of the sequence are
// gathered on the host into pinned memory (the embedding itself never moves
// to the device), the blocks run back to back on device buffers through
// mamba_block_forward's device-pointer path, and the head product
// logits[L, V] = h[L, D] . head[D, V] (the reference's gemm_f32,
// kernels/gemm_f32.c:13-31) runs on the fp32 matrix cores. The head goes
// up and the logits come down through the runtime's pinned ring (host memcpy
// on a thread pool overlapping the DMA); the product runs in chunks of rows
// so the download of the first rows overlaps the rest of the product.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "km_device.hpp"
#include "../km_runtime.hpp"
#include "kmamba.h"
#include "kmamba_km.h"

namespace km {

typedef float f32x16 __attribute__((ext_vector_type(16)));

// C[M, N] = A[M, K] . B[K, N], all row-major fp32, on
// v_mfma_f32_32x32x2_f32. A workgroup of four waves owns a 64x64 tile of C
// (each wave a 32x32 quarter) and walks K in steps of 16 through LDS,
// double-buffered: the next step's elements are loaded into registers while
// the current step's eight MFMAs per wave run. Loads are scalar and lane
// order follows memory order (16 lanes per 64-byte A row segment, 64 lanes
// per 256-byte B row segment); elements past M, N or K load as zero through
// the buffer range check or an out-of-range offset. A is stored k-major in
// LDS so a lane's operand (row l%32, k l/32) is a conflict-free read.
constexpr int kHM = 64, kHN = 64, kHK = 16;

__global__ void __launch_bounds__(256) lm_head_f32(const float *__restrict__ A,
                                                   const float *__restrict__ B, float *__restrict__ Cm,
                                                   long M, long K, long N) {
    __shared__ float sA[2][kHK][kHM + 4];
    __shared__ float sB[2][kHK][kHN + 4];
    constexpr unsigned kDrop = 0x80000000u;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = w >> 1, wn = w & 1;
    const long m0 = static_cast<long>(blockIdx.y) * kHM, n0 = static_cast<long>(blockIdx.x) * kHN;
    const long arows = std::min<long>(kHM, M - m0);
    const long bcols = std::min<long>(kHN, N - n0);
    // Windows: A rows m0.. (K floats each), B rows k.. of the tile's columns.
    const auto rA = make_rsrc(A + m0 * K, arows * K * 4);
    const auto rB = make_rsrc(B + n0, ((K - 1) * N + bcols) * 4);
    float ra[4], rb[4];
    auto load = [&](long k0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = tid + 256 * i;
            const int am = e / kHK, ak = e % kHK;              // A: 16 lanes per row segment
            const bool ain = am < arows && k0 + ak < K;
            const unsigned oa = ain ? static_cast<unsigned>((am * K + k0 + ak) * 4) : kDrop;
            ra[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rA, oa, 0, 0));
            const int bk = e / kHN, bn = e % kHN;              // B: 64 lanes per row segment
            const bool bin = bn < bcols && k0 + bk < K;
            const unsigned ob = bin ? static_cast<unsigned>(((k0 + bk) * N + bn) * 4) : kDrop;
            rb[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rB, ob, 0, 0));
        }
    };
    auto store = [&](int s) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = tid + 256 * i;
            sA[s][e % kHK][e / kHK] = ra[i];
            sB[s][e / kHN][e % kHN] = rb[i];
        }
    };
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
    const int fr = lane & 31, fk = lane >> 5;
    const long nk = (K + kHK - 1) / kHK;
    load(0);
    store(0);
    __syncthreads();
    for (long kt = 0; kt < nk; ++kt) {
        const int s = static_cast<int>(kt & 1);
        if (kt + 1 < nk) load((kt + 1) * kHK);
#pragma unroll
        for (int kk = 0; kk < kHK / 2; ++kk) {
            const float a = sA[s][2 * kk + fk][wm * 32 + fr];
            const float b = sB[s][2 * kk + fk][wn * 32 + fr];
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc, 0, 0, 0);
        }
        if (kt + 1 < nk) store(s ^ 1);
        __syncthreads();
    }
    // Lane l holds rows 8*(r/4) + 4*(l/32) + r%4, column l%32 of the quarter.
    const long col = n0 + wn * 32 + fr;
    if (col >= N) return;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const long row = m0 + wm * 32 + 8 * (r >> 2) + 4 * fk + (r & 3);
        if (row < M) Cm[row * N + col] = acc[r];
    }
}

static int lm_head_launch(const float *A, const float *B, float *C, long M, long K, long N,
                          hipStream_t s) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    // 32-bit byte offsets inside the A and B windows.
    if (static_cast<double>(kHM) * K * 4 > 2147483647.0 || static_cast<double>(K) * N * 4 > 2147483647.0) {
        set_error("kmamba_forward: head of %ld x %ld too large for 32-bit offsets", K, N);
        return -1;
    }
    const long gx = (N + kHN - 1) / kHN, gy = (M + kHM - 1) / kHM;
    if (gx > 0x7fffffffL || gy > 65535) {
        set_error("kmamba_forward: head grid %ld x %ld out of range", gx, gy);
        return -1;
    }
    hipLaunchKernelGGL(lm_head_f32, dim3(static_cast<unsigned>(gx), static_cast<unsigned>(gy)),
                       dim3(256), 0, s, A, B, C, M, K, N);
    KM_HIP_TRY(hipGetLastError());
    return 0;
}

// Rows of the head product per launch on the download pipeline (each launch
// reads the whole head; 256 rows keep that re-read small against the product).
constexpr size_t kHeadChunkRows = 256;

// Events without timing, destroyed with the set.
class EventSet {
  public:
    explicit EventSet(size_t n) : ev_(n, nullptr) {
        for (auto &e : ev_)
            if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
                (void)hipGetLastError();
                e = nullptr;
                ok_ = false;
                set_error("kmamba_forward: hipEventCreate failed");
            }
    }
    ~EventSet() {
        for (auto e : ev_)
            if (e) (void)hipEventDestroy(e);
    }
    EventSet(const EventSet &) = delete;
    EventSet &operator=(const EventSet &) = delete;
    bool ok() const { return ok_; }
    hipEvent_t operator[](size_t i) const { return ev_[i]; }

  private:
    std::vector<hipEvent_t> ev_;
    bool ok_ = true;
};

// 80-byte checkpoint header of version 4 (ref src/kmamba.c:216-229).
struct CkptHeader {
    char magic[8];
    uint32_t version;
    uint32_t reserved;
    uint64_t vocab_size;
    uint64_t dim;
    uint64_t state_size;
    uint64_t seq_len;
    uint64_t n_layers;
    uint64_t mimo_rank;
    float dt_scale;
    float dt_min;
    float dt_max;
};
static_assert(sizeof(CkptHeader) == 80, "checkpoint header is 80 bytes");

// The block parameters in checkpoint order (ref src/kmamba.c:262-273).
struct BlockArrays {
    float *p[10];
    size_t n[10];
};
static BlockArrays block_arrays(MambaBlock *b) {
    const size_t ts = b->config.state_size / 2 > 0 ? b->config.state_size / 2 : 1;
    BlockArrays a{{b->W_in.data, b->W_out.data, b->A_log.data, b->W_B.data, b->W_C.data, b->b_B,
                   b->b_C, b->delta_proj.data, b->lambda_proj.data, b->theta},
                  {b->W_in.rows * b->W_in.cols, b->W_out.rows * b->W_out.cols,
                   b->A_log.rows * b->A_log.cols, b->W_B.rows * b->W_B.cols,
                   b->W_C.rows * b->W_C.cols, b->W_B.rows, b->W_C.rows,
                   b->delta_proj.rows * b->delta_proj.cols,
                   b->lambda_proj.rows * b->lambda_proj.cols, ts}};
    return a;
}

static void xavier_uniform(float *w, size_t fan_in, size_t fan_out, size_t n) {
    // ref src/kmamba.c:19-27: the same float expressions and rand() order.
    const float scale = sqrtf(6.0f / (static_cast<float>(fan_in) + static_cast<float>(fan_out)));
    for (size_t i = 0; i < n; i++)
        w[i] = (static_cast<float>(rand()) / static_cast<float>(RAND_MAX) * 2.0f - 1.0f) * scale;
}

}  // namespace km

extern "C" {

KMamba *kmamba_create(const KMambaConfig *cfg) {
    km::clear_error();
    if (!cfg || !cfg->vocab_size || !cfg->dim || !cfg->seq_len || !cfg->n_layers) {
        km::set_error("kmamba_create: vocab_size, dim, seq_len and n_layers must be non-zero");
        return nullptr;
    }
    KMamba *m = static_cast<KMamba *>(calloc(1, sizeof(KMamba)));
    if (!m) {
        km::set_error("kmamba_create: out of memory");
        return nullptr;
    }
    m->cfg = *cfg;
    if (km_normalize_spatial_topology(&m->cfg.spatial_ndims, m->cfg.spatial_dims, m->cfg.seq_len,
                                      m->cfg.use_convnd, &m->cfg.convnd_ndims, m->cfg.convnd_K) != 0) {
        free(m);
        km::set_error("kmamba_create: invalid spatial topology");
        return nullptr;
    }
    const size_t VD = m->cfg.vocab_size * m->cfg.dim;
    m->embedding = static_cast<float *>(calloc(VD, sizeof(float)));
    m->head = m->cfg.weight_tying ? m->embedding : static_cast<float *>(calloc(VD, sizeof(float)));
    m->layers = static_cast<MambaBlock **>(calloc(m->cfg.n_layers, sizeof(MambaBlock *)));
    if (!m->embedding || !m->head || !m->layers) {
        kmamba_free(m);
        km::set_error("kmamba_create: out of memory");
        return nullptr;
    }
    for (size_t i = 0; i < m->cfg.n_layers; i++) {
        MBConfig bc{};
        bc.dim = m->cfg.dim;
        bc.state_size = m->cfg.state_size;
        bc.seq_len = m->cfg.seq_len;
        bc.mimo_rank = m->cfg.mimo_rank > 0 ? m->cfg.mimo_rank : 1;
        bc.dt_scale = m->cfg.dt_scale;
        bc.dt_min = m->cfg.dt_min;
        bc.dt_max = m->cfg.dt_max;
        bc.spatial_ndims = m->cfg.spatial_ndims;
        bc.use_convnd = m->cfg.use_convnd;
        bc.convnd_K = m->cfg.convnd_K;
        bc.convnd_ndims = m->cfg.convnd_ndims;
        memcpy(bc.spatial_dims, m->cfg.spatial_dims, sizeof(bc.spatial_dims));
        m->layers[i] = mamba_block_create(&bc);
        if (!m->layers[i]) {
            kmamba_free(m);
            km::set_error("kmamba_create: block %zu could not be created", i);
            return nullptr;
        }
    }
    return m;
}

void kmamba_free(KMamba *m) {
    if (!m) return;
    if (m->layers) {
        for (size_t i = 0; i < m->cfg.n_layers; i++) mamba_block_free(m->layers[i]);
        free(m->layers);
    }
    if (m->head != m->embedding) free(m->head);
    free(m->embedding);
    free(m->m_embedding);
    free(m->v_embedding);
    free(m->m_head);
    free(m->v_head);
    free(m);
}

int kmamba_init(KMamba *m, uint32_t seed) {
    if (!m) return -1;
    srand(static_cast<unsigned>(seed));
    const size_t V = m->cfg.vocab_size, D = m->cfg.dim;
    km::xavier_uniform(m->embedding, V, D, V * D);
    if (!m->cfg.weight_tying) km::xavier_uniform(m->head, D, V, D * V);
    for (size_t i = 0; i < m->cfg.n_layers; i++) mamba_block_init(m->layers[i]);
    return 0;
}

int kmamba_save(const KMamba *m, const char *path) {
    km::clear_error();
    if (!m || !path) {
        km::set_error("kmamba_save: NULL argument");
        return -1;
    }
    FILE *f = fopen(path, "wb");
    if (!f) {
        km::set_error("kmamba_save: cannot open %s", path);
        return -1;
    }
    km::CkptHeader h;
    memset(&h, 0, sizeof(h));
    memcpy(h.magic, "KMAMBA", 6);
    h.version = 4;
    h.vocab_size = m->cfg.vocab_size;
    h.dim = m->cfg.dim;
    h.state_size = m->cfg.state_size;
    h.seq_len = m->cfg.seq_len;
    h.n_layers = m->cfg.n_layers;
    h.mimo_rank = m->cfg.mimo_rank > 0 ? m->cfg.mimo_rank : 1;
    h.dt_scale = m->cfg.dt_scale;
    h.dt_min = m->cfg.dt_min;
    h.dt_max = m->cfg.dt_max;
    const size_t VD = m->cfg.vocab_size * m->cfg.dim;
    bool ok = fwrite(&h, sizeof(h), 1, f) == 1 && fwrite(m->embedding, sizeof(float), VD, f) == VD &&
              fwrite(m->head, sizeof(float), VD, f) == VD;
    for (size_t i = 0; ok && i < m->cfg.n_layers; i++) {
        const km::BlockArrays a = km::block_arrays(m->layers[i]);
        for (int j = 0; ok && j < 10; ++j) ok = fwrite(a.p[j], sizeof(float), a.n[j], f) == a.n[j];
    }
    ok = (fclose(f) == 0) && ok;
    if (!ok) {
        km::set_error("kmamba_save: write to %s failed", path);
        return -1;
    }
    return 0;
}

KMamba *kmamba_load(const char *path, int for_training, const MBOptimConfig *opt_blocks,
                    float lr_embed_head, float weight_decay) {
    (void)opt_blocks;
    (void)lr_embed_head;
    (void)weight_decay;
    km::clear_error();
    if (!path) {
        km::set_error("kmamba_load: NULL path");
        return nullptr;
    }
    if (for_training) {
        km::set_error("kmamba_load: training is not part of this library (for_training must be 0)");
        return nullptr;
    }
    FILE *f = fopen(path, "rb");
    if (!f) {
        km::set_error("kmamba_load: cannot open %s", path);
        return nullptr;
    }
    km::CkptHeader h;
    if (fread(&h, sizeof(h), 1, f) != 1 || memcmp(h.magic, "KMAMBA", 6) != 0 || h.version > 4) {
        fclose(f);
        km::set_error("kmamba_load: %s is not a checkpoint of version <= 4", path);
        return nullptr;
    }
    KMambaConfig cfg{};
    cfg.vocab_size = h.vocab_size;
    cfg.dim = h.dim;
    cfg.state_size = h.state_size;
    cfg.seq_len = h.seq_len;
    cfg.n_layers = h.n_layers;
    cfg.mimo_rank = (h.version >= 4 && h.mimo_rank > 0) ? h.mimo_rank : 1;
    cfg.dt_scale = h.dt_scale;
    cfg.dt_min = h.dt_min;
    cfg.dt_max = h.dt_max;
    KMamba *m = kmamba_create(&cfg);
    if (!m) {
        fclose(f);
        return nullptr;
    }
    const size_t VD = cfg.vocab_size * cfg.dim;
    bool ok = fread(m->embedding, sizeof(float), VD, f) == VD && fread(m->head, sizeof(float), VD, f) == VD;
    for (size_t i = 0; ok && i < cfg.n_layers; i++) {
        const km::BlockArrays a = km::block_arrays(m->layers[i]);
        for (int j = 0; ok && j < 10; ++j) ok = fread(a.p[j], sizeof(float), a.n[j], f) == a.n[j];
    }
    fclose(f);
    if (!ok) {
        kmamba_free(m);
        km::set_error("kmamba_load: %s is truncated", path);
        return nullptr;
    }
    return m;
}

int kmamba_forward(KMamba *m, const uint32_t *tokens, float *logits_out) {
    km::clear_error();
    if (!m || !tokens || !logits_out) {
        km::set_error("kmamba_forward: NULL argument");
        return -1;
    }
    const size_t L = m->cfg.seq_len, D = m->cfg.dim, V = m->cfg.vocab_size;
    const size_t N = m->cfg.state_size;
    for (size_t i = 0; i < m->cfg.n_layers; i++) {
        memset(m->layers[i]->hidden, 0, N * sizeof(float));
        memset(m->layers[i]->scan_h, 0, N * sizeof(float));
    }
    if (!km::gpu_ready()) return -1;
    // Device buffers: two activation buffers, the head and the logits.
    const size_t act = km::align_up(sizeof(float) * L * D, 256);
    const size_t hb = km::align_up(sizeof(float) * D * V, 256);
    const size_t lb = km::align_up(sizeof(float) * L * V, 256);
    char *ws = static_cast<char *>(km::Workspace::reserve(2 * act + hb + lb, nullptr, km::WsUse::Model));
    if (!ws) return -1;
    float *buf[2] = {reinterpret_cast<float *>(ws), reinterpret_cast<float *>(ws + act)};
    float *dhead = reinterpret_cast<float *>(ws + 2 * act);
    float *dlog = reinterpret_cast<float *>(ws + 2 * act + hb);
    // Embedding rows of the sequence (ref src/kmamba.c:85-98), gathered on
    // the host into pinned memory and sent in one copy.
    km::Staging::lock();
    float *pin = static_cast<float *>(km::PinnedStaging::reserve(sizeof(float) * L * D));
    bool ok = pin != nullptr;
    if (ok) {
        (void)hipStreamSynchronize(nullptr);     // no earlier copy still reads the pinned block
        const size_t per = 64;   // rows per task of the host thread pool
        km::host_parallel_for((L + per - 1) / per, [&](size_t i) {
            for (size_t t = i * per; t < std::min(L, (i + 1) * per); t++) {
                if (tokens[t] < V) memcpy(pin + t * D, m->embedding + static_cast<size_t>(tokens[t]) * D, D * sizeof(float));
                else memset(pin + t * D, 0, D * sizeof(float));
            }
        });
        ok = hipMemcpyAsync(buf[0], pin, sizeof(float) * L * D, hipMemcpyHostToDevice, nullptr) == hipSuccess &&
             hipStreamSynchronize(nullptr) == hipSuccess;
        if (!ok) km::set_error("kmamba_forward: embedding upload failed");
    }
    km::Staging::unlock();
    if (!ok) return -1;
    // The head is host memory the caller owns (and may change between calls),
    // so it goes up on every call, through the pinned ring, on a helper
    // thread while this one runs the blocks (which do not touch dhead). The
    // thread is joined before the head product; errors come back by value
    // since the error message is per thread.
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        km::set_error("kmamba_forward: no current HIP device");
        return -1;
    }
    int up_rc = 0;
    std::string up_err;
    std::thread up([&] {
        if (hipSetDevice(dev) != hipSuccess) {
            up_rc = -1;
            up_err = "kmamba_forward: hipSetDevice failed on the upload thread";
            return;
        }
        up_rc = km::host_pipe_upload(dhead, m->head, sizeof(float) * D * V, nullptr);
        if (up_rc != 0) up_err = km_last_error();
    });
    int cur = 0;
    bool blocks_ok = true;
    for (size_t i = 0; blocks_ok && i < m->cfg.n_layers; i++) {
        mamba_block_forward(m->layers[i], buf[cur ^ 1], buf[cur], 1);
        blocks_ok = km_last_error()[0] == '\0';
        cur ^= 1;
    }
    up.join();
    if (!blocks_ok) return -1;
    if (up_rc != 0) {
        km::set_error("%s", up_err.c_str());
        return -1;
    }
    // The head product in chunks of rows, each followed by an event: a piece
    // of the logits goes down as soon as the chunk holding its last row is
    // written, while later chunks are computed.
    const size_t rows = km::kHeadChunkRows;
    km::EventSet ev((L + rows - 1) / rows);
    if (!ev.ok()) return -1;
    for (size_t c = 0; c * rows < L; ++c) {
        const size_t r0 = c * rows, nr = std::min(rows, L - r0);
        if (km::lm_head_launch(buf[cur] + r0 * D, dhead, dlog + r0 * V, static_cast<long>(nr),
                               static_cast<long>(D), static_cast<long>(V), nullptr) != 0)
            return -1;
        if (hipEventRecord(ev[c], nullptr) != hipSuccess) {
            km::set_error("kmamba_forward: hipEventRecord failed");
            return -1;
        }
    }
    return km::host_pipe_download(logits_out, dlog, sizeof(float) * L * V, sizeof(float) * V,
                                  [&](size_t end_row) { return ev[(end_row - 1) / rows]; });
}

}  // extern "C"
