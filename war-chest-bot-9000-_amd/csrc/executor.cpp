// Executor: weight banks, wave upload and the CFR schedule on one HIP stream.
// The schedule follows engine/src/gpu/device.rs:641-718 (initialise, the
// iteration loop with snapshots, Phase 2 per carried root).
#include "executor.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <unordered_map>

#include "../../include/wc_wave.h"
#include "check.h"
#include "par.h"

namespace wc {

namespace {

#define HIP_TRY(expr)                                                       \
    do {                                                                    \
        hipError_t e_ = (expr);                                             \
        if (e_ != hipSuccess) {                                             \
            if (err) *err = std::string(#expr ": ") + hipGetErrorString(e_); \
            return false;                                                   \
        }                                                                   \
    } while (0)

// `t^p / (t^p + 1)` with the infinities evaluated (engine/src/search.rs:185-193).
float cfr_factor(float t, float p) {
    if (std::isinf(p)) return p > 0.0f ? 1.0f : 0.0f;
    float x = std::pow(t, p);
    return x / (x + 1.0f);
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// The table blob: arrays at 256-byte aligned offsets, laid out first, then
// copied into pinned staging memory on several host threads (the upload is one
// asynchronous copy from there). The sources must outlive copy_to.
struct Blob {
    struct Piece {
        const uint8_t* src;
        size_t bytes, at;
    };
    std::vector<Piece> pieces;
    size_t size = 0;
    template <class T>
    size_t put(const std::vector<T>& v) {
        const size_t at = align256(size), bytes = v.size() * sizeof(T);
        if (bytes) pieces.push_back({(const uint8_t*)v.data(), bytes, at});
        size = at + std::max<size_t>(bytes, 4);
        return at;
    }
    void copy_to(uint8_t* dst) const {
        constexpr size_t CHUNK = size_t(8) << 20;
        std::vector<Piece> parts;  // pieces cut into chunks of at most CHUNK bytes
        for (const Piece& pc : pieces)
            for (size_t o = 0; o < pc.bytes; o += CHUNK)
                parts.push_back({pc.src + o, std::min(CHUNK, pc.bytes - o), pc.at + o});
        parallel_for(
            parts.size(), [&](size_t k) { std::memcpy(dst + parts[k].at, parts[k].src, parts[k].bytes); }, 8);
    }
};

}  // namespace

Executor::Executor(int device, int precision) : device_(device), precision_(precision) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
        err_ = "no HIP device";
        return;
    }
    if (device < 0 || device >= n) {
        err_ = "device index out of range";
        return;
    }
    if (precision < WC_PRECISE || precision > WC_F16X) {
        err_ = "unknown precision";
        return;
    }
    if (hipSetDevice(device) != hipSuccess || hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking) != hipSuccess ||
        hipStreamCreateWithFlags(&copy_, hipStreamNonBlocking) != hipSuccess) {
        err_ = "cannot create the executor streams";
        return;
    }
    void* flag = nullptr;
    if (hipHostMalloc(&flag, 256, hipHostMallocDefault) != hipSuccess) {
        err_ = "cannot allocate the executor's pinned flag";
        return;
    }
    check_host_ = (uint32_t*)flag;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && cus > 0)
        cus_ = (uint32_t)cus;
    for (Slot& sl : slots_)
        if (hipEventCreateWithFlags(&sl.uploaded, hipEventDisableTiming) != hipSuccess ||
            hipEventCreateWithFlags(&sl.done, hipEventDisableTiming) != hipSuccess ||
            hipEventRecord(sl.done, stream_) != hipSuccess) {  // (an upload waits on it: complete at once)
            err_ = "cannot create the executor's events";
            return;
        }
    if (!noalloc_scratch(device, &scratch_, &scratch_err_)) scratch_ = nullptr;
    if (const char* env = std::getenv("WC_CHAIN_SPLIT")) split_ = std::strcmp(env, "0") != 0;
    if (const char* env = std::getenv("WC_GRAPH")) graph_ = std::strcmp(env, "1") == 0;
    if (const char* env = std::getenv("WC_UNIT_LDS")) unit_lds_ = std::strcmp(env, "0") != 0;
    if (const char* env = std::getenv("WC_V5_SCALAR")) v5_scalar_ = std::strcmp(env, "1") == 0;
    ok_ = true;
}

Executor::~Executor() {
    if (!stream_) return;
    hipSetDevice(device_);
    hipStreamSynchronize(stream_);
    if (copy_) hipStreamSynchronize(copy_);
    for (auto& kv : banks_) hipFree(kv.second.mem);
    for (void* t : table_) hipFree(t);
    hipFree(arena_);
    hipFree(mlp_);
    for (Slot& sl : slots_) {
        if (sl.pin) hipHostFree(sl.pin);
        if (sl.res) hipHostFree(sl.res);
        if (sl.uploaded) hipEventDestroy(sl.uploaded);
        if (sl.done) hipEventDestroy(sl.done);
        if (sl.exec) hipGraphExecDestroy(sl.exec);
    }
    if (check_host_) hipHostFree(check_host_);
    if (copy_) hipStreamDestroy(copy_);
    hipStreamDestroy(stream_);
}

bool Executor::ensure(void** p, size_t* cap, size_t need, std::string* err) {
    if (need <= *cap && *p) return true;
    if (*p) {
        HIP_TRY(hipStreamSynchronize(stream_));
        HIP_TRY(hipStreamSynchronize(copy_));
        HIP_TRY(hipFree(*p));
        *p = nullptr;
    }
    size_t sz = 1;
    while (sz < need) sz <<= 1;  // power-of-two reservation, as the reference's arena
    HIP_TRY(hipMalloc(p, sz));
    *cap = sz;
    return true;
}

// Grow-only pinned host staging (a power-of-two reservation, like the device
// buffers); the stream is drained before a buffer is replaced.
bool Executor::ensure_pinned(uint8_t** p, size_t* cap, size_t need, std::string* err) {
    if (need <= *cap && *p) return true;
    if (*p) {
        HIP_TRY(hipStreamSynchronize(stream_));
        HIP_TRY(hipStreamSynchronize(copy_));
        HIP_TRY(hipHostFree(*p));
        *p = nullptr;
        *cap = 0;
    }
    size_t sz = 1;
    while (sz < need) sz <<= 1;
    void* q = nullptr;
    HIP_TRY(hipHostMalloc(&q, sz, hipHostMallocDefault));
    *p = (uint8_t*)q;
    *cap = sz;
    return true;
}

uint64_t Executor::publish_v5(const NetShape& ns, const float* w, size_t nw, const float* b, size_t nb,
                              const float* ln, size_t nln, std::string* err) {
    const v5::Layout L = v5::layout();
    if (nw != L.w_len || nb != L.b_len || nln != L.ln_len || !w || !b || !ln) {
        *err = "v5 weight bank sizes disagree with net.rs's layout (w " + std::to_string(L.w_len) + ", b " +
               std::to_string(L.b_len) + ", ln " + std::to_string(L.ln_len) + ")";
        return 0;
    }
    if (precision_ == WC_F16X) {
        *err = "compensated f16 takes the MLP leaf network only";
        return 0;
    }
    if (hipSetDevice(device_) != hipSuccess) {
        *err = "hipSetDevice failed";
        return 0;
    }
    // One allocation: the f32 blob (matrices, biases, norms), the board
    // tables, and for the 16-bit path each matrix-core GEMM's B operand
    // (fragment-major, one K-contiguous row per output, K padded to whole
    // 32-column steps with zeros, rows padded to GEMM_ROWS) with the f32
    // staging it is converted from.
    const v5::Board bd = v5::board();
    const size_t o_w = 0, o_b = align256(nw * 4), o_ln = o_b + align256(nb * 4), o_bd = o_ln + align256(nln * 4);
    size_t total = o_bd + align256(sizeof bd);
    const bool mfma = (precision_ == WC_F16 || precision_ == WC_BF16) && !v5_scalar_;
    size_t o_m16[v5::M_COUNT] = {}, o_stage = 0, stage_floats = 0;
    std::vector<float> stage;
    if (mfma) {
        for (uint32_t m = 0; m < v5::M_COUNT; m++) {
            const v5::Span sp = v5::mat_span(L, m);
            o_m16[m] = total;
            total += align256(size_t(gemm_rows(sp.o)) * v5::kpad(sp.i) * 2);
            stage_floats += size_t(v5::kpad(sp.i)) * sp.o;
        }
        o_stage = total;
        total += align256(stage_floats * 4);
        stage.assign(stage_floats, 0.0f);
        size_t at = 0;
        for (uint32_t m = 0; m < v5::M_COUNT; m++) {  // [kpad(i) x o], rows past i zero
            const v5::Span sp = v5::mat_span(L, m);
            std::copy(w + sp.w, w + sp.w + size_t(sp.i) * sp.o, stage.begin() + at);
            at += size_t(v5::kpad(sp.i)) * sp.o;
        }
    }
    void* mem = nullptr;
    if (hipMalloc(&mem, total) != hipSuccess) {
        *err = "hipMalloc of the weight bank failed";
        return 0;
    }
    char* base = (char*)mem;
    bool okc = hipMemcpyAsync(base + o_w, w, nw * 4, hipMemcpyHostToDevice, stream_) == hipSuccess &&
               hipMemcpyAsync(base + o_b, b, nb * 4, hipMemcpyHostToDevice, stream_) == hipSuccess &&
               hipMemcpyAsync(base + o_ln, ln, nln * 4, hipMemcpyHostToDevice, stream_) == hipSuccess &&
               hipMemcpyAsync(base + o_bd, &bd, sizeof bd, hipMemcpyHostToDevice, stream_) == hipSuccess;
    if (mfma) {
        okc = okc && hipMemsetAsync(base + o_m16[0], 0, o_stage - o_m16[0], stream_) == hipSuccess &&
              hipMemcpyAsync(base + o_stage, stage.data(), stage_floats * 4, hipMemcpyHostToDevice, stream_) ==
                  hipSuccess;
        size_t at = 0;
        for (uint32_t m = 0; m < v5::M_COUNT && okc; m++) {
            const v5::Span sp = v5::mat_span(L, m);
            launch_to16(precision_, (const float*)(base + o_stage) + at, base + o_m16[m], sp.o, v5::kpad(sp.i), true,
                        stream_);
            at += size_t(v5::kpad(sp.i)) * sp.o;
        }
    }
    okc = okc && hipStreamSynchronize(stream_) == hipSuccess && hipGetLastError() == hipSuccess;
    if (!okc) {
        hipFree(mem);
        *err = "weight upload failed";
        return 0;
    }
    NetBank bank;
    bank.ns = ns;
    bank.precision = precision_;
    bank.mem = mem;
    bank.v5.w = (const float*)(base + o_w);
    bank.v5.b = (const float*)(base + o_b);
    bank.v5.ln = (const float*)(base + o_ln);
    bank.v5.nb = (const uint8_t*)(base + o_bd) + offsetof(v5::Board, nb);
    bank.v5.loc = (const uint8_t*)(base + o_bd) + offsetof(v5::Board, loc);
    bank.v5.value_bias = b[L.value_bias];
    if (mfma)
        for (uint32_t m = 0; m < v5::M_COUNT; m++) bank.v5.m16[m] = (const uint16_t*)(base + o_m16[m]);
    bank.version = next_version_++;
    banks_[bank.version] = bank;
    return bank.version;
}

uint64_t Executor::publish(const NetShape& ns, const std::vector<uint32_t>& dims, const float* w, size_t nw,
                           const float* b, size_t nb, std::string* err, const float* ln, size_t nln) {
    if (ns.kind == MODEL_V5) return publish_v5(ns, w, nw, b, nb, ln, nln, err);
    if (nln) {
        *err = "the synthetic networks take no LayerNorm parameters";
        return 0;
    }
    const bool tower = ns.kind == MODEL_TWO_TOWER;
    if (ns.kind != MODEL_MLP && !tower) {
        *err = "this executor builds the MLP and two-tower leaf networks only";
        return 0;
    }
    if (ns.layers == 0 || ns.layers > 15 || (tower && (ns.priv_layers == 0 || ns.priv_layers > 15))) {
        *err = "network depth out of range";
        return 0;
    }
    // Source matrices in `w` order, (K, N) each: the MLP's trunk then head
    // ([heads x hidden], one row per output); the two-tower's public then
    // private tower, then the readout weight vector.
    struct Mat {
        size_t k, n;
        bool head;
    };
    std::vector<Mat> mats;
    mats.push_back({ns.in, ns.hidden, false});
    for (uint32_t l = 1; l < ns.layers; l++) mats.push_back({ns.hidden, ns.hidden, false});
    if (tower) {
        mats.push_back({ns.priv_in, ns.hidden, false});
        for (uint32_t l = 1; l < ns.priv_layers; l++) mats.push_back({ns.hidden, ns.hidden, false});
    } else {
        mats.push_back({ns.hidden, ns.heads, true});
    }
    size_t need_w = tower ? ns.hidden : 0;
    for (const Mat& m : mats) need_w += m.k * m.n;
    const size_t need_b = tower ? size_t(ns.layers + ns.priv_layers) * ns.hidden + 1
                                : size_t(ns.layers) * ns.hidden + ns.heads;
    if (nw != need_w || nb != need_b) {
        *err = "weight bank sizes disagree with dims";
        return 0;
    }
    if (tower && precision_ == WC_F16X) {
        *err = "compensated f16 takes the MLP leaf network only";
        return 0;
    }
    if (precision_ != WC_PRECISE && (ns.in % 32 || ns.hidden % 32 || (tower && (ns.priv_in % 32 || ns.hidden > 512)))) {
        *err = tower ? "the MFMA path needs input, private-input and width multiples of 32 (width at most 512)"
                     : "the MFMA path needs input and hidden widths that are multiples of 32";
        return 0;
    }
    if (hipSetDevice(device_) != hipSuccess) {
        *err = "hipSetDevice failed";
        return 0;
    }
    NetBank bank;
    bank.ns = ns;
    bank.precision = precision_;
    // Bytes per stored matrix element: float32, one 16-bit value, or the
    // compensated pair (hi and lo planes).
    const size_t esz = precision_ == WC_PRECISE ? 4 : precision_ == WC_F16X ? 4 : 2;
    // Layout: matrices (as stored for the arithmetic), then f32 biases, then
    // the two-tower readout weight. The exact net keeps the source layout; the
    // MFMA net stores each matrix as the GEMM's B operand (one row per output,
    // K-contiguous), fragment-major with gemm_rows(N) zero-padded rows.
    std::vector<size_t> moff;
    size_t at = 0;
    auto stored_bytes = [&](const Mat& m) {
        if (precision_ == WC_PRECISE) return m.k * m.n * esz;
        return size_t(gemm_rows((uint32_t)m.n)) * m.k * esz;
    };
    for (const Mat& m : mats) {
        moff.push_back(at);
        at = align256(at + stored_bytes(m));
    }
    const size_t mats_end = at;
    const size_t boff = at;
    at = align256(at + nb * 4);
    const size_t roff = at;  // readout weight (two-tower), f32
    if (tower) at = align256(at + size_t(ns.hidden) * 4);
    // Staging for f32 -> 16-bit conversion on the device.
    const size_t stage = precision_ == WC_PRECISE ? 0 : at;
    const size_t total = at + (precision_ == WC_PRECISE ? 0 : nw * 4);
    void* mem = nullptr;
    if (hipMalloc(&mem, total) != hipSuccess) {
        *err = "hipMalloc of the weight bank failed";
        return 0;
    }
    char* base = (char*)mem;
    bool okc = hipMemcpyAsync(base + boff, b, nb * 4, hipMemcpyHostToDevice, stream_) == hipSuccess;
    size_t src = 0;
    if (precision_ == WC_PRECISE) {
        for (size_t k = 0; k < mats.size(); k++) {
            const size_t n = mats[k].k * mats[k].n;
            okc = okc && hipMemcpyAsync(base + moff[k], w + src, n * 4, hipMemcpyHostToDevice, stream_) == hipSuccess;
            src += n;
        }
    } else {
        okc = okc && hipMemsetAsync(base, 0, mats_end, stream_) == hipSuccess;  // row padding
        okc = okc && hipMemcpyAsync(base + stage, w, nw * 4, hipMemcpyHostToDevice, stream_) == hipSuccess;
        for (size_t k = 0; k < mats.size(); k++) {
            const size_t n = mats[k].k * mats[k].n;
            // Trunk and tower matrices are [K x N] (B row n = source column n);
            // the MLP head is [N x K] (one K-contiguous row per output).
            launch_to16(precision_, (const float*)(base + stage) + src, base + moff[k], (uint32_t)mats[k].n,
                        (uint32_t)mats[k].k, !mats[k].head, stream_);
            src += n;
        }
    }
    if (tower)
        okc = okc && hipMemcpyAsync(base + roff, w + src, size_t(ns.hidden) * 4, hipMemcpyHostToDevice, stream_) ==
                         hipSuccess;
    okc = okc && hipStreamSynchronize(stream_) == hipSuccess && hipGetLastError() == hipSuccess;
    if (!okc) {
        hipFree(mem);
        *err = "weight upload failed";
        return 0;
    }
    bank.mem = mem;
    for (uint32_t l = 0; l < ns.layers; l++) {
        bank.W[l] = base + moff[l];
        bank.B[l] = (const float*)(base + boff) + size_t(l) * ns.hidden;
    }
    if (tower) {
        for (uint32_t l = 0; l < ns.priv_layers; l++) {
            bank.PW[l] = base + moff[ns.layers + l];
            bank.PB[l] = (const float*)(base + boff) + size_t(ns.layers + l) * ns.hidden;
        }
        bank.wread = (const float*)(base + roff);
        bank.bread = b[size_t(ns.layers + ns.priv_layers) * ns.hidden];
    } else {
        bank.Whead = base + moff[ns.layers];
        bank.bhead = (const float*)(base + boff) + size_t(ns.layers) * ns.hidden;
    }
    bank.version = next_version_++;
    (void)dims;
    banks_[bank.version] = bank;
    return bank.version;
}

void Executor::retain_from(uint64_t oldest) {
    hipSetDevice(device_);
    for (auto it = banks_.begin(); it != banks_.end();) {
        if (it->first < oldest) {
            hipStreamSynchronize(stream_);
            hipFree(it->second.mem);
            it = banks_.erase(it);
        } else {
            ++it;
        }
    }
}

bool Executor::upload(const WaveHost& w, const NetBank& bank, uint32_t slot, std::string* err, bool device_check,
                      std::function<void()>* meanwhile) {
    const NetShape& ns = bank.ns;
    device_check = device_check || !w.checked;
    if (device_check && !validate_shape(w, err)) return false;  // before the sizes below are trusted
    if (w.net.kind != ns.kind || w.net.in != ns.in || w.net.hidden != ns.hidden || w.net.pool != ns.pool ||
        w.net.heads != ns.heads || w.net.layers != ns.layers || w.net.priv_in != ns.priv_in ||
        w.net.priv_layers != ns.priv_layers) {
        *err = "wave network shape disagrees with the weight bank";
        return false;
    }
    HIP_TRY(hipSetDevice(device_));
    Blob blob;
    struct Off {
        size_t node_meta, nc, legal_value, draw_to, draw_p, reach_base, vals_base, rev_src, rev_cell, rvd_src, rvd_p,
            row_node, row_cfg_off, row_cfg, cfg_emb, pub_raw, term_node, term_util, roots, carried, exit_node,
            exit_coff, exit_reach, trees, units, bt[2], rt[2], dc[2], bl[2], rl[2], cv[2], lr[2], pg[2], twb[2], twu[2], cfg_priv,
            unit_term, tb[2], tr[2], tc[2], rc[2], rp[2], head_tile_n, cp[2], card_feat, row_job, cfg_job, cfg_owner;
    } o;
    o.node_meta = blob.put(w.node_meta);
    o.nc = blob.put(w.node_nc);
    o.legal_value = blob.put(w.legal_value);
    o.draw_to = blob.put(w.draw_to);
    o.draw_p = blob.put(w.draw_p);
    o.reach_base = blob.put(w.reach_base);
    o.vals_base = blob.put(w.vals_base);
    o.rev_src = blob.put(w.rev_src);
    o.rev_cell = blob.put(w.rev_cell);
    o.rvd_src = blob.put(w.rvd_src);
    o.rvd_p = blob.put(w.rvd_p);
    o.row_node = blob.put(w.row_node);
    o.row_cfg_off = blob.put(w.row_cfg_off);
    o.row_cfg = blob.put(w.row_cfg);
    o.cfg_emb = blob.put(w.cfg_emb);
    o.cfg_priv = blob.put(w.cfg_priv);
    o.card_feat = blob.put(w.card_feat);
    o.row_job = blob.put(w.row_job);
    o.cfg_job = blob.put(w.cfg_job);
    o.cfg_owner = blob.put(w.cfg_owner);
    o.pub_raw = blob.put(w.pub_raw);
    o.term_node = blob.put(w.term_node);
    o.term_util = blob.put(w.term_util);
    o.roots = blob.put(w.roots);
    o.carried = blob.put(w.carried);
    o.exit_node = blob.put(w.exit_node);
    o.exit_coff = blob.put(w.exit_coff);
    o.exit_reach = blob.put(w.exit_reach);
    o.trees = blob.put(w.trees);
    o.units = blob.put(w.units);
    for (int p = 0; p < 2; p++) {
        o.bt[p] = blob.put(w.back_rec[p]);
        o.rt[p] = blob.put(w.reach_rec[p]);
        o.dc[p] = blob.put(w.acc_rec[p]);
        o.cv[p] = blob.put(w.child_vb[p]);
        o.lr[p] = blob.put(w.leaf_rec[p]);
        o.pg[p] = blob.put(w.pool_grp[p]);
        o.twb[p] = blob.put(w.tower_blk[p]);
        o.twu[p] = blob.put(w.tower_unit[p]);
        o.bl[p] = blob.put(w.back_lvl[p]);
        o.rl[p] = blob.put(w.reach_lvl[p]);
    }
    o.unit_term = blob.put(w.unit_term);
    o.head_tile_n = blob.put(w.head_tile_n);
    std::vector<ChainPass> plan[2];
    for (int p = 0; p < 2; p++) {
        plan[p] = plan_chain(w.head_rb_n[p].data(), (uint32_t)w.head_rb_n[p].size(), w.net.heads, cus_);
        if (!check_chain_plan(plan[p], w.head_rb_n[p].data(), (uint32_t)w.head_rb_n[p].size(), w.net.heads, err))
            return false;
        o.cp[p] = blob.put(plan[p]);
        chain_npass_[p] = (uint32_t)plan[p].size();
    }
    for (int p = 0; p < 2; p++) {
        o.tb[p] = blob.put(w.top_back_rec[p]);
        o.tr[p] = blob.put(w.top_reach_rec[p]);
        o.tc[p] = blob.put(w.top_back_chunk[p]);
        o.rc[p] = blob.put(w.top_reach_chunk[p]);
        o.rp[p] = blob.put(w.top_reach_par[p]);
    }
    // The device check's words follow the tables: it runs beside the wave
    // before, which holds the solve state.
    const size_t check_at = align256(blob.size), check_words = 1 + 2 * size_t(w.rows());
    if (!ensure(&table_[slot], &table_cap_[slot], check_at + check_words * 4, err)) return false;
    Slot& sl = slots_[slot];
    if (sl.recorded) HIP_TRY(hipEventSynchronize(sl.uploaded));  // the slot's last upload has left its staging
    if (!ensure_pinned(&sl.pin, &sl.pin_cap, blob.size, err)) return false;
    blob.copy_to(sl.pin);
    HIP_TRY(hipStreamWaitEvent(copy_, sl.done, 0));  // the slot's last wave no longer reads its tables
    HIP_TRY(hipMemcpyAsync(table_[slot], sl.pin, blob.size, hipMemcpyHostToDevice, copy_));
    HIP_TRY(hipEventRecord(sl.uploaded, copy_));  // (recorded again below, after the check)
    sl.recorded = true;

    // Mutable arena.
    const size_t cells = std::max<uint32_t>(w.ncells, 1), rl = std::max<uint32_t>(w.reach_len, 1),
                 vl = std::max<uint32_t>(w.vals_len, 1), rows = w.rows();
    size_t at = 0;
    auto take = [&](size_t bytes) {
        size_t a = align256(at);
        at = a + std::max<size_t>(bytes, 4);
        return a;
    };
    size_t a_regret = take(cells * 4), a_cur = take(cells * 4), a_sum = take(cells * 4), a_snap = take(cells * 4);
    size_t a_reach = take(rl * 4), a_sreach = take(rl * 4), a_vals = take(vl * 4);
    size_t a_mass = take(rows * 2 * 4);
    size_t a_roots = take(size_t(w.root_values_len) * 4);
    size_t a_carry = take(size_t(w.carry_slots) * w.snapshot_configs * 2);
    if (!ensure(&arena_, &arena_cap_, at, err)) return false;
    // Leaf-network activations (compensated f16: hi and lo planes, 4 bytes per element).
    const size_t esz = precision_ == WC_PRECISE || precision_ == WC_F16X ? 4 : 2;
    size_t mt = 0;
    auto mtake = [&](size_t bytes) {
        size_t a = align256(mt);
        mt = a + std::max<size_t>(bytes, 4);
        return a;
    };
    const size_t prow = precision_ == WC_PRECISE ? rows : gemm_rows((uint32_t)rows);  // GEMM operands: padded rows
    const bool tower = ns.kind == MODEL_TWO_TOWER, v5net = ns.kind == MODEL_V5;
    const size_t ncfg = w.cfg_key.size(), pcfg = precision_ == WC_PRECISE ? ncfg : gemm_rows((uint32_t)ncfg);
    // Query-input width: the v5 join's 129 columns padded to whole k steps as a 16-bit operand.
    const size_t xin = v5net && precision_ != WC_PRECISE ? v5::JOIN_IN_PAD : ns.in;
    size_t m_x = mtake(prow * xin * esz), m_x1 = mtake(prow * xin * esz), m_h0 = mtake(prow * ns.hidden * esz),
           m_h1 = mtake(prow * ns.hidden * esz),
           m_out = mtake(readout_net(ns.kind) ? w.tower_len * 4 : rows * ns.heads * 4);
    // The fused net's first-layer product over the fixed query columns, when
    // the pooled columns are whole 32-column k steps ahead of them.
    const bool split = split_ && ns.kind == MODEL_MLP && (precision_ == WC_F16 || precision_ == WC_BF16) &&
                       chain_fits(ns.in, ns.hidden, ns.layers) && ns.pool > 0 && ns.in > 2 * ns.pool &&
                       (2 * ns.pool) % 32 == 0;
    size_t m_s0 = split ? mtake(prow * ns.hidden * 4) : 0, m_s1 = split ? mtake(prow * ns.hidden * 4) : 0;
    size_t m_px = 0, m_p0 = 0, m_p1 = 0, m_f = 0;
    if (tower) {
        m_px = mtake(precision_ == WC_PRECISE ? 0 : pcfg * ns.priv_in * esz);
        m_p0 = mtake(pcfg * ns.hidden * esz);
        m_p1 = mtake(pcfg * ns.hidden * esz);
        m_f = mtake(ncfg * ns.hidden * esz);
    }
    // v5: cards and bag rows per job, P and Jp per row, g and f per config, the join's input scratch.
    const size_t njobs = w.trees.size();
    size_t m_cards = 0, m_bag = 0, m_P = 0, m_Jp = 0, m_G = 0, m_F = 0, m_xf = 0;
    if (v5net) {
        m_cards = mtake(njobs * 2 * v5::NTYPE * v5::TYPE * 4);
        m_bag = mtake(njobs * 2 * v5::NTYPE * 3 * v5::POOL * 4);
        m_P = mtake(rows * v5::D * 4);
        m_Jp = mtake(rows * v5::JW * 4);
        m_G = mtake(ncfg * v5::POOL * 4);
        m_F = mtake(ncfg * v5::D * esz);
        m_xf = mtake(precision_ == WC_PRECISE ? 0 : rows * v5::JOIN_IN * 4);
    }
    if (!ensure(&mlp_, &mlp_cap_, mt, err)) return false;

    char* T = (char*)table_[slot];
    check_ = (uint32_t*)(T + check_at);
    char* A = (char*)arena_;
    char* M = (char*)mlp_;
    WaveDev& d = dev_;
    d = WaveDev{};
    d.node_meta = (const uint32_t*)(T + o.node_meta);
    d.nc = (const uint32_t*)(T + o.nc);
    d.legal_value = (const uint32_t*)(T + o.legal_value);
    d.draw_to = (const uint32_t*)(T + o.draw_to);
    d.draw_p = (const float*)(T + o.draw_p);
    d.reach_base = (const uint32_t*)(T + o.reach_base);
    d.vals_base = (const uint32_t*)(T + o.vals_base);
    d.rev_src = (const uint32_t*)(T + o.rev_src);
    d.rev_cell = (const uint32_t*)(T + o.rev_cell);
    d.rvd_src = (const uint32_t*)(T + o.rvd_src);
    d.rvd_p = (const float*)(T + o.rvd_p);
    d.row_node = (const uint32_t*)(T + o.row_node);
    d.row_cfg_off = (const uint32_t*)(T + o.row_cfg_off);
    d.row_cfg = (const uint32_t*)(T + o.row_cfg);
    d.cfg_emb = (const float*)(T + o.cfg_emb);
    d.pub_raw = (const uint8_t*)(T + o.pub_raw);
    d.term_node = (const uint32_t*)(T + o.term_node);
    d.term_util = (const float*)(T + o.term_util);
    d.roots = (const float*)(T + o.roots);
    d.carried = (const float*)(T + o.carried);
    d.exit_node = (const uint32_t*)(T + o.exit_node);
    d.exit_coff = (const uint32_t*)(T + o.exit_coff);
    d.exit_reach = (const uint32_t*)(T + o.exit_reach);
    d.trees = (const TreeDev*)(T + o.trees);
    d.units = (const UnitDev*)(T + o.units);
    for (int p = 0; p < 2; p++) {
        d.back_rec[p] = (const BackRec*)(T + o.bt[p]);
        d.reach_rec[p] = (const ReachRec*)(T + o.rt[p]);
        d.acc_rec[p] = (const AccRec*)(T + o.dc[p]);
        d.child_vb[p] = (const uint32_t*)(T + o.cv[p]);
        d.leaf_rec[p] = (const LeafRec*)(T + o.lr[p]);
        d.pool_grp[p] = (const PoolGroup*)(T + o.pg[p]);
        d.npool[p] = (uint32_t)w.pool_grp[p].size();
        d.nleaf[p] = (uint32_t)w.leaf_rec[p].size();
        d.tower_blk[p] = (const TowerBlock*)(T + o.twb[p]);
        d.tower_unit[p] = (const TowerUnit*)(T + o.twu[p]);
        d.ntower_blk[p] = (uint32_t)w.tower_blk[p].size();
        d.ntower_unit[p] = (uint32_t)w.tower_unit[p].size();
        d.back_lvl[p] = (const uint32_t*)(T + o.bl[p]);
        d.reach_lvl[p] = (const uint32_t*)(T + o.rl[p]);
        d.ndec[p] = (uint32_t)w.decision[p].size();
    }
    d.unit_term = (const uint32_t*)(T + o.unit_term);
    head_tile_n_ = (const uint32_t*)(T + o.head_tile_n);
    for (int p = 0; p < 2; p++) chain_plan_[p] = (const ChainPass*)(T + o.cp[p]);
    for (int p = 0; p < 2; p++) {
        top_back_dev_[p] = (const BackRec*)(T + o.tb[p]);
        top_reach_dev_[p] = (const ReachRec*)(T + o.tr[p]);
        top_chunk_dev_[p] = (const uint32_t*)(T + o.tc[p]);
        top_reach_chunk_dev_[p] = (const uint32_t*)(T + o.rc[p]);
        top_reach_par_dev_[p] = (const uint32_t*)(T + o.rp[p]);
    }
    d.nunits = (uint32_t)w.units.size();
    d.max_vwin = w.max_vwin;
    d.max_rwin = w.max_rwin;
    d.unit_lds = unit_lds_ ? 1u : 0u;
    d.nsub = w.nsub;
    d.regret = (float*)(A + a_regret);
    d.cur = (float*)(A + a_cur);
    d.sum = (float*)(A + a_sum);
    d.snap = (float*)(A + a_snap);
    d.reach = (float*)(A + a_reach);
    d.snap_reach = (float*)(A + a_sreach);
    d.vals = (float*)(A + a_vals);
    d.mass = (float*)(A + a_mass);
    d.root_values = (float*)(A + a_roots);
    d.carry = (uint16_t*)(A + a_carry);
    d.ntrees = (uint32_t)w.trees.size();
    d.rows = w.rows();
    d.pool = ns.pool;
    d.in = (uint32_t)xin;
    d.row_bytes = v5net ? 0 : ns.row_bytes;  // v5: the public bytes feed the trunk, not the query input
    d.snapshot_configs = w.snapshot_configs;
    d.xplane = uint64_t(prow) * xin;
    d.nexit = (uint32_t)w.exit_node.size();
    d.ncells = w.ncells;
    X_ = M + m_x;
    Xq_[0] = M + m_x;
    Xq_[1] = M + m_x1;
    H_[0] = M + m_h0;
    H_[1] = M + m_h1;
    S_[0] = split ? (float*)(M + m_s0) : nullptr;
    S_[1] = split ? (float*)(M + m_s1) : nullptr;
    head_out_ = (float*)(M + m_out);
    cfg_priv_ = (const float*)(T + o.cfg_priv);
    PX_ = tower ? M + m_px : nullptr;
    P_[0] = tower ? M + m_p0 : nullptr;
    P_[1] = tower ? M + m_p1 : nullptr;
    F_ = tower ? M + m_f : nullptr;
    ncfg_ = tower ? (uint32_t)ncfg : 0;
    rows_ = w.rows();
    v5_in_ = v5::WaveIn{};
    v5_out_ = v5::WaveOut{};
    v5_xf_ = nullptr;
    if (v5net) {
        v5_in_.jobs = (uint32_t)njobs;
        v5_in_.rows = (uint32_t)rows;
        v5_in_.ncfg = (uint32_t)ncfg;
        v5_in_.card_feat = (const float*)(T + o.card_feat);
        v5_in_.raw = (const uint8_t*)(T + o.pub_raw);
        v5_in_.row_job = (const uint32_t*)(T + o.row_job);
        v5_in_.phi = (const float*)(T + o.cfg_priv);
        v5_in_.cfg_job = (const uint32_t*)(T + o.cfg_job);
        v5_in_.cfg_owner = (const uint8_t*)(T + o.cfg_owner);
        v5_out_.cards = (float*)(M + m_cards);
        v5_out_.bag = (float*)(M + m_bag);
        v5_out_.P = (float*)(M + m_P);
        v5_out_.Jp = (float*)(M + m_Jp);
        v5_out_.G = (float*)(M + m_G);
        v5_out_.F = M + m_F;
        v5_xf_ = precision_ == WC_PRECISE ? nullptr : (float*)(M + m_xf);
        d.cfg_emb = v5_out_.G;  // the pooled beliefs pool g(c) (search.rs:1525-1545)
    }
    if (device_check && !check_on_device(w, err, meanwhile)) return false;
    HIP_TRY(hipEventRecord(sl.uploaded, copy_));
    HIP_TRY(hipStreamWaitEvent(stream_, sl.uploaded, 0));  // the schedule reads the tables once they are in
    launch_query_static(d, precision_, Xq_[0], Xq_[1], stream_);
    HIP_TRY(hipGetLastError());
    return true;
}

bool Executor::check_on_device(const WaveHost& w, std::string* err, std::function<void()>* meanwhile) {
    if (w.max_rwin > CHECK_RWIN_MAX) return validate_deep(w, err);  // wider than the unit check's bitmap
    // On the upload's stream, behind the tables' copy and beside the wave
    // before; the host waits only for the copy and the check.
    launch_zero((float*)check_, 1 + 2 * size_t(w.rows()), copy_);
    launch_check(check_args(w, dev_, top_back_dev_, top_reach_dev_, check_, check_ + 1), copy_);
    HIP_TRY(hipGetLastError());
    *check_host_ = 0;
    HIP_TRY(hipMemcpyAsync(check_host_, check_, sizeof(uint32_t), hipMemcpyDeviceToHost, copy_));
    if (meanwhile && *meanwhile) {
        const std::function<void()> f = std::move(*meanwhile);
        *meanwhile = nullptr;
        f();
    }
    HIP_TRY(hipStreamSynchronize(copy_));
    const uint32_t flag = *(volatile uint32_t*)check_host_;
    if (flag) {
        const char* m = check_message(CHECK_BASE - flag);
        *err = std::string("wave bounds: ") + (m ? m : "unknown condition");
        return false;
    }
    return true;
}

bool Executor::check(const WaveHost& w, uint64_t version, std::string* err) {
    const NetBank* bank = bank_of(version, err);
    if (!bank) return false;
    if (in_flight_) {
        *err = "collect the launched waves before checking";
        return false;
    }
    HIP_TRY(hipSetDevice(device_));
    if (!upload(w, *bank, 0, err, true)) return false;
    HIP_TRY(hipStreamSynchronize(stream_));
    return true;
}

ChainNet chain_net(const NetBank& bank) {
    const NetShape& ns = bank.ns;
    ChainNet net{};
    for (uint32_t l = 0; l < ns.layers; l++) {
        net.w[l] = (const uint16_t*)bank.W[l];
        net.b[l] = bank.B[l];
    }
    net.w[ns.layers] = (const uint16_t*)bank.Whead;
    net.b[ns.layers] = bank.bhead;
    net.in = ns.in;
    net.hidden = ns.hidden;
    net.layers = ns.layers;
    net.heads = ns.heads;
    return net;
}

void Executor::run_mlp(const NetBank& bank, uint32_t rows, const void* x, std::vector<hipEvent_t>* marks,
                       const uint32_t* head_tile_n, const ChainPass* plan, uint32_t npass, const float* part) {
    const NetShape& ns = bank.ns;
    auto mark = [&]() {
        if (marks) {
            hipEvent_t e;
            hipEventCreate(&e);
            hipEventRecord(e, stream_);
            marks->push_back(e);
        }
    };
    if ((precision_ == WC_F16 || precision_ == WC_BF16) && chain_fits(ns.in, ns.hidden, ns.layers)) {
        ChainNet net = chain_net(bank);
        if (part) {
            net.part = part;
            net.dsteps = 2 * ns.pool / 32;
        }
        launch_chain(precision_, net, x, rows, head_out_, plan, npass, stream_);
        mark();
        return;
    }
    const void* in = x;
    uint32_t k = ns.in;
    for (uint32_t l = 0; l < ns.layers; l++) {
        void* out = H_[l & 1];
        if (precision_ == WC_PRECISE)
            launch_dense_exact((const float*)in, k, (const float*)bank.W[l], bank.B[l], ns.hidden, (float*)out, rows,
                               stream_);
        else
            launch_gemm16(precision_, in, k, bank.W[l], bank.B[l], ns.hidden, out, rows, true, true, stream_);
        mark();
        in = out;
        k = ns.hidden;
    }
    if (precision_ == WC_PRECISE)
        launch_head_exact((const float*)in, ns.hidden, (const float*)bank.Whead, bank.bhead, ns.heads, head_out_,
                          rows, stream_);
    else
        launch_gemm16(precision_, in, ns.hidden, bank.Whead, bank.bhead, ns.heads, head_out_, rows, false, false,
                      stream_, head_tile_n);
    mark();
}

void Executor::run_tower_private(const NetBank& bank) {
    const NetShape& ns = bank.ns;
    if (!ncfg_) return;
    const void* in = cfg_priv_;
    uint32_t k = ns.priv_in;
    if (precision_ != WC_PRECISE) {
        launch_to16(precision_, cfg_priv_, PX_, ncfg_, ns.priv_in, false, stream_);
        in = PX_;
    }
    for (uint32_t l = 0; l < ns.priv_layers; l++) {
        void* out = P_[l & 1];
        if (precision_ == WC_PRECISE)
            launch_dense_exact((const float*)in, k, (const float*)bank.PW[l], bank.PB[l], ns.hidden, (float*)out,
                               ncfg_, stream_);
        else
            launch_gemm16(precision_, in, k, bank.PW[l], bank.PB[l], ns.hidden, out, ncfg_, true, true, stream_);
        in = out;
        k = ns.hidden;
    }
    launch_tower_f(precision_, in, ns.hidden, ncfg_, bank.wread, F_, stream_);
}

void Executor::run_tower(const NetBank& bank, uint32_t rows, int traverser) {
    const NetShape& ns = bank.ns;
    const void* in = Xq_[traverser];
    uint32_t k = ns.in;
    for (uint32_t l = 0; l < ns.layers; l++) {
        void* out = H_[l & 1];
        if (precision_ == WC_PRECISE)
            launch_dense_exact((const float*)in, k, (const float*)bank.W[l], bank.B[l], ns.hidden, (float*)out, rows,
                               stream_);
        else
            launch_gemm16(precision_, in, k, bank.W[l], bank.B[l], ns.hidden, out, rows, true, true, stream_);
        in = out;
        k = ns.hidden;
    }
    launch_tower_head(dev_, traverser, precision_, in, ns.hidden, F_, bank.bread, head_out_, stream_);
}

const NetBank* Executor::bank_of(uint64_t version, std::string* err) const {
    auto it = banks_.find(version);
    if (it == banks_.end()) {
        *err = "GPU weight version " + std::to_string(version) + " is unavailable";
        return nullptr;
    }
    return &it->second;
}

void Executor::run_v5_build(const NetBank& bank) { v5::launch_build(precision_, bank.v5, v5_in_, v5_out_, stream_); }

void Executor::run_v5_join(const NetBank& bank, int traverser) {
    v5::launch_join(precision_, bank.v5, dev_.rows, Xq_[traverser], v5_out_.P, v5_out_.Jp, H_[0], v5_xf_, stream_);
}

void Executor::run_v5_readout(const NetBank& bank, int traverser) {
    launch_tower_head(dev_, traverser, precision_, H_[0], v5::D, v5_out_.F, bank.v5.value_bias, head_out_, stream_);
}

void Executor::run_v5(const NetBank& bank, int traverser) {
    run_v5_join(bank, traverser);
    run_v5_readout(bank, traverser);
}

void Executor::leaf_net(const NetBank& bank, int q) {
    if (bank.ns.kind == MODEL_V5)
        run_v5(bank, q);
    else if (bank.ns.kind == MODEL_TWO_TOWER)
        run_tower(bank, dev_.rows, q);
    else
        run_mlp(bank, dev_.rows, Xq_[q], nullptr, head_tile_n_, chain_plan_[q], chain_npass_[q], S_[q]);
}

// Top regions' values bottom-up, one launch per run of the wave's plan: one
// depth, or two whose dependent rows the packer grouped into chunks.
void Executor::top_back(const WaveHost& w, int p, int mode, float da, float db, float pr) {
    const std::vector<uint32_t>& run = w.top_back_run[p];
    for (size_t i = 0; i < run.size(); i += TOP_RUN) {
        const uint32_t l = run[i];
        if (run[i + 1] == NONE) {
            const uint32_t b = w.top_back_lvl[p][l], e = w.top_back_lvl[p][l + 1];
            launch_back_rows(dev_, top_back_dev_[p] + b, e - b, p, mode, da, db, pr, stream_);
        } else {
            launch_back_pair(dev_, top_back_dev_[p], top_chunk_dev_[p] + run[i + 2], run[i + 3], p, mode, da, db, pr,
                             stream_);
        }
    }
}

// Top regions' reach, top-down, one launch per depth at which a run of the
// wave's plan starts (one depth, or two chunk by chunk); p < 0: both players.
// With reach2 (p >= 0), the launches also take both players' rows under
// strat2 into reach2 (an independent reach computation). The sets are
// independent, so each follows its own runs.
void Executor::top_reach(const WaveHost& w, int p, float* reach, const float* strat, float* reach2,
                         const float* strat2) {
    struct Set {
        int q;
        float* reach;
        const float* strat;
        size_t next;  // the set's next run
    } sets[3];
    int ns = 0;
    for (int q = 0; q < 2; q++)
        if (p < 0 || p == q) sets[ns++] = Set{q, reach, strat, 0};
    if (reach2 && p >= 0)
        for (int q = 0; q < 2; q++) sets[ns++] = Set{q, reach2, strat2, 0};
    for (uint32_t l = 0; l < w.top_levels; l++) {
        ReachSet one[3];
        ReachPair two[3] = {};
        int n1 = 0, n2 = 0;
        for (int i = 0; i < ns; i++) {
            Set& s = sets[i];
            const std::vector<uint32_t>& run = w.top_reach_run[s.q];
            if (s.next >= run.size() || run[s.next] != l) continue;
            if (run[s.next + 1] == NONE) {
                const uint32_t b = w.top_reach_lvl[s.q][l], n = w.top_reach_lvl[s.q][l + 1] - b;
                one[n1++] = ReachSet{top_reach_dev_[s.q] + b, n, s.reach, s.strat};
            } else {
                two[n2++] = ReachPair{top_reach_dev_[s.q], top_reach_chunk_dev_[s.q] + run[s.next + 2],
                                      top_reach_par_dev_[s.q], run[s.next + 3], s.reach, s.strat};
            }
            s.next += TOP_RUN;
        }
        if (n1) launch_reach_rows(dev_, one[0], one[1], one[2], stream_);
        if (n2) launch_reach_pair(dev_, two[0], two[1], two[2], stream_);
    }
}

// Both players' reach under a fixed strategy: tops first, then their subtrees.
void Executor::reach_both(const WaveHost& w, float* reach, const float* strat) {
    top_reach(w, -1, reach, strat);
    launch_reach(dev_, 0, w.nsub, reach, strat, -1, stream_);
}

// The first layer's product over each traverser's fixed query columns, under
// this bank (when the fused net runs with the split).
void Executor::static_products(const NetBank& bank) {
    if (!S_[0]) return;
    ChainNet net = chain_net(bank);
    net.dsteps = 2 * bank.ns.pool / 32;  // the pooled columns come first; the rest are fixed
    for (int q = 0; q < 2; q++) launch_chain_static(precision_, net, Xq_[q], S_[q], chain_plan_[q], chain_npass_[q], stream_);
}

// Solver::new on the device (engine/src/search.rs:826-888): uniform strategy,
// zero regret, reach from the root beliefs, the seeded average sums, the first
// carries, and both players' leaf inputs.
void Executor::init_state(const WaveHost& w) {
    const WaveDev& d = dev_;
    hipStream_t s = stream_;
    launch_zero(d.regret, w.ncells, s);
    launch_init_strategy(d, s);
    launch_seed_reach(d, d.reach, w.reach_len, -1, s);
    reach_both(w, d.reach, d.cur);
    launch_seed_sum(d, s);
    if (w.carry_slots) launch_gather_carry(d, d.reach, 0, s);
    launch_pool(d, -1, precision_, Xq_[0], Xq_[1], s);
}

void Executor::run_schedule(const WaveHost& w, const NetBank& bank, ScheduleTimes* prof, const LeafHook* hook) {
    const WaveDev& d = dev_;
    hipStream_t s = stream_;
    const Meta& m = w.meta;
    const uint32_t nsub = w.nsub;
    // Per-class attribution: an event after every launch group, binned by class.
    // C_BUILD (the per-wave network work) and C_JOIN (the v5 join) count as
    // leaf-net time and are also reported on their own.
    enum { C_BACK = 0, C_TOP = 1, C_REACH = 2, C_MLP = 3, C_LEAF = 4, C_OTHER = 5, C_BUILD = 6, C_JOIN = 7 };
    std::vector<std::pair<hipEvent_t, int>> ev;
    hipEvent_t start = nullptr;
    auto mark = [&](int cls) {
        if (!prof) return;
        hipEvent_t e;
        hipEventCreate(&e);
        hipEventRecord(e, s);
        ev.push_back({e, cls});
    };
    if (prof) {
        hipEventCreate(&start);
        hipEventRecord(start, s);
    }
    const bool tower = bank.ns.kind == MODEL_TWO_TOWER;
    if (tower) {
        run_tower_private(bank);  // F for this wave's configs under this bank
        mark(C_BUILD);
    }
    if (bank.ns.kind == MODEL_V5) {
        run_v5_build(bank);  // cards, trunk, configs for this wave under this bank
        mark(C_BUILD);
    }
    if (S_[0]) {
        static_products(bank);
        mark(C_BUILD);
    }
    // One traverser's leaf net; under profiling the v5 join is timed apart from its readout.
    auto net_pass = [&](int p) {
        if (prof && bank.ns.kind == MODEL_V5) {
            run_v5_join(bank, p);
            mark(C_JOIN);
            run_v5_readout(bank, p);
        } else {
            leaf_net(bank, p);
        }
    };
    init_state(w);
    mark(C_OTHER);
    int carry_pending = -1;  // a snapshot whose carries the next iteration's reach launches compute
    if (m.iters == 0) launch_normalize(d, 0, 0, s);
    for (uint32_t t = 0; t < m.iters; t++) {
        const int p = (int)(t & 1);
        net_pass(p);
        if (hook) (*hook)((int32_t)t, p);
        mark(C_MLP);
        const float mm = (float)(t / 2 + 1);
        const float da = cfr_factor(mm, m.cfr.alpha), db = cfr_factor(mm, m.cfr.beta);
        const float ds = std::pow(mm / (mm + 1.0f), m.cfr.gamma);
        launch_sweep(d, 0, nsub, head_out_, bank.ns.heads, p, MODE_REGRET, da, db, m.cfr.predict, s);
        mark(C_BACK);
        top_back(w, p, MODE_REGRET, da, db, m.cfr.predict);
        // A snapshot's carried beliefs (both players' reach under the average
        // strategy, then the gather) ride in this iteration's reach launches:
        // the average strategy does not change before the next snapshot,
        // which is normalised after them.
        float* snap_reach = carry_pending >= 0 ? d.snap_reach : nullptr;
        top_reach(w, p, d.reach, d.cur, snap_reach, d.snap);
        mark(C_TOP);
        launch_reach(d, 0, nsub, d.reach, d.cur, p, s, snap_reach, d.snap);
        if (carry_pending >= 0) launch_gather_carry(d, d.snap_reach, carry_pending, s);
        carry_pending = -1;
        mark(C_REACH);
        launch_pool(d, p, precision_, Xq_[0], Xq_[1], s, p, ds);  // with p's average accumulation
        mark(C_LEAF);
        const uint32_t done = t + 1;
        auto it = std::find(m.snap_iters.begin(), m.snap_iters.end(), done);
        if (it != m.snap_iters.end() && (m.snapshots || done == m.iters)) {
            size_t si = size_t(it - m.snap_iters.begin());
            launch_normalize(d, 1, done >= 2 ? 1 : 0, s);
            if (m.snapshots && si + 1 < m.snap_iters.size()) {
                launch_seed_reach(d, d.snap_reach, w.reach_len, -1, s);
                if (done < m.iters) {
                    carry_pending = (int)si;  // in the next iteration's reach launches
                } else {
                    reach_both(w, d.snap_reach, d.snap);
                    launch_gather_carry(d, d.snap_reach, (int)si, s);
                }
            }
            mark(C_OTHER);
        }
    }
    // Phase 2: root values under the final average for every carried root.
    for (uint32_t root = 0; root < w.nroots_max; root++) {
        launch_seed_reach(d, d.reach, w.reach_len, (int)root, s);
        reach_both(w, d.reach, d.snap);
        mark(C_OTHER);
        launch_pool(d, -1, precision_, Xq_[0], Xq_[1], s);
        mark(C_LEAF);
        for (int p = 0; p < 2; p++) {
            net_pass(p);
            if (hook) (*hook)(phase2_point(root, p), p);
            launch_sweep(d, 0, nsub, head_out_, bank.ns.heads, p, MODE_VALUE, 0.0f, 0.0f, 0.0f, s);
            top_back(w, p, MODE_VALUE, 0.0f, 0.0f, 0.0f);
            launch_collect_root(d, (int)root, p, s);
            mark(C_OTHER);
        }
    }
    if (prof) {
        hipStreamSynchronize(s);
        *prof = ScheduleTimes{};
        hipEvent_t prev = start;
        double cls_ms[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        uint32_t cls_n[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (auto& e : ev) {
            float ms = 0.0f;
            hipEventElapsedTime(&ms, prev, e.first);
            cls_ms[e.second] += ms;
            cls_n[e.second]++;
            prev = e.first;
        }
        float tot = 0.0f;
        if (!ev.empty()) hipEventElapsedTime(&tot, start, ev.back().first);
        prof->total = tot;
        prof->cfr = cls_ms[C_BACK] + cls_ms[C_TOP] + cls_ms[C_REACH];
        prof->mlp = cls_ms[C_MLP] + cls_ms[C_BUILD] + cls_ms[C_JOIN];
        prof->net_build = cls_ms[C_BUILD];
        prof->v5_join = cls_ms[C_JOIN];
        prof->leaf_input = cls_ms[C_LEAF];
        prof->other = cls_ms[C_OTHER];
        prof->back_mean = cls_n[C_BACK] ? cls_ms[C_BACK] / cls_n[C_BACK] : 0.0;
        prof->top_mean = cls_n[C_TOP] ? cls_ms[C_TOP] / cls_n[C_TOP] : 0.0;
        prof->reach_mean = cls_n[C_REACH] ? cls_ms[C_REACH] / cls_n[C_REACH] : 0.0;
        prof->cfr_launches = cls_n[C_BACK];
        prof->cfr_launch_mean = cls_n[C_BACK] ? prof->cfr / cls_n[C_BACK] : 0.0;
        for (auto& e : ev) hipEventDestroy(e.first);
        hipEventDestroy(start);
    }
}

bool Executor::capture(const WaveHost& w, const NetBank& bank, hipGraphExec_t* exec, double* build_ms,
                       std::string* err) {
    const auto t0 = std::chrono::steady_clock::now();
    HIP_TRY(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
    run_schedule(w, bank, nullptr);
    hipGraph_t g = nullptr;
    HIP_TRY(hipStreamEndCapture(stream_, &g));
    const hipError_t e = hipGraphInstantiate(exec, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (e != hipSuccess) {
        *err = std::string("hipGraphInstantiate: ") + hipGetErrorString(e);
        return false;
    }
    if (build_ms)
        *build_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    return true;
}

bool Executor::launch(const WaveHost& w, uint64_t version, InFlight* f, std::string* err,
                      const std::function<void()>& meanwhile) {
    std::function<void()> pending = meanwhile;  // called once: during the device check, else at the end
    const bool ok = launch_wave(w, version, f, err, &pending);
    if (pending) pending();
    return ok;
}

bool Executor::launch_wave(const WaveHost& w, uint64_t version, InFlight* f, std::string* err,
                           std::function<void()>* meanwhile) {
    const NetBank* bank = bank_of(version, err);
    if (!bank) return false;
    if (f->live) {
        *err = "this in-flight record holds a wave that was not collected";
        return false;
    }
    // The lowest free slot: a caller that collects each wave before launching
    // the next keeps reusing one slot's pinned buffers.
    uint32_t k = MAX_IN_FLIGHT;
    for (uint32_t i = 0; i < MAX_IN_FLIGHT; i++)
        if (!slots_[i].busy) {
            k = i;
            break;
        }
    if (k == MAX_IN_FLIGHT) {
        *err = "the executor already has " + std::to_string(MAX_IN_FLIGHT) + " waves in flight; collect one first";
        return false;
    }
    Slot& sl = slots_[k];
    // Reserved from here (`meanwhile` may collect the other slot during the
    // upload); released again on every failure below.
    struct Reserve {
        Slot& s;
        bool keep = false;
        ~Reserve() {
            if (!keep) s.busy = false;
        }
    } reserve{sl};
    sl.busy = true;
    if (!upload(w, *bank, k, err, false, meanwhile)) return false;
    if (sl.exec) {
        HIP_TRY(hipGraphExecDestroy(sl.exec));
        sl.exec = nullptr;
    }
    if (graph_) {
        if (!capture(w, *bank, &sl.exec, nullptr, err)) return false;
        HIP_TRY(hipGraphLaunch(sl.exec, stream_));
    } else {
        run_schedule(w, *bank, nullptr);
    }
    HIP_TRY(hipGetLastError());
    // The outputs go into the slot's pinned landing, in the stream after the schedule.
    const size_t ns_ = w.ncells, nr = w.root_values_len, nc = size_t(w.carry_slots) * w.snapshot_configs;
    const size_t o_roots = align256(ns_ * 4), o_carry = o_roots + align256(nr * 4);
    if (!ensure_pinned(&sl.res, &sl.res_cap, o_carry + nc * 2 + 4, err)) return false;
    if (ns_) HIP_TRY(hipMemcpyAsync(sl.res, dev_.snap, ns_ * 4, hipMemcpyDeviceToHost, stream_));
    if (nr) HIP_TRY(hipMemcpyAsync(sl.res + o_roots, dev_.root_values, nr * 4, hipMemcpyDeviceToHost, stream_));
    if (nc) HIP_TRY(hipMemcpyAsync(sl.res + o_carry, dev_.carry, nc * 2, hipMemcpyDeviceToHost, stream_));
    HIP_TRY(hipEventRecord(sl.done, stream_));
    f->slot = k;
    f->version = version;
    f->ncells = ns_;
    f->nroots = nr;
    f->carry_slots = w.carry_slots;
    f->snapshot_configs = w.snapshot_configs;
    f->o_roots = o_roots;
    f->o_carry = o_carry;
    f->jobs.resize(w.jobs.size());
    for (size_t j = 0; j < w.jobs.size(); j++) {
        const TreeDev& t = w.trees[j];
        JobSlice& js = f->jobs[j];
        js.ncells = w.jobs[j]->t.ncells;
        js.nroots = t.nroots;
        js.n0 = t.n0;
        js.n1 = t.n1;
        js.root_value0 = t.root_value0;
        js.snapshot_configs = w.jobs[j]->t.snapshot_configs();
    }
    reserve.keep = true;
    in_flight_++;
    f->live = true;
    return true;
}

bool Executor::trim(std::string* err) {
    if (in_flight_) {
        *err = "cannot trim with waves in flight";
        return false;
    }
    HIP_TRY(hipSetDevice(device_));
    HIP_TRY(hipStreamSynchronize(stream_));
    HIP_TRY(hipStreamSynchronize(copy_));
    for (uint32_t k = 0; k < MAX_IN_FLIGHT; k++) {
        HIP_TRY(hipFree(table_[k]));
        table_[k] = nullptr;
        table_cap_[k] = 0;
    }
    HIP_TRY(hipFree(arena_));
    HIP_TRY(hipFree(mlp_));
    arena_ = mlp_ = nullptr;
    arena_cap_ = mlp_cap_ = 0;
    for (Slot& sl : slots_) {
        if (sl.pin) HIP_TRY(hipHostFree(sl.pin));
        if (sl.res) HIP_TRY(hipHostFree(sl.res));
        sl.pin = sl.res = nullptr;
        sl.pin_cap = sl.res_cap = 0;
    }
    rows_ = 0;
    return true;
}

bool Executor::ready(const InFlight& f) const {
    return f.live && hipEventQuery(slots_[f.slot].done) == hipSuccess;
}

// Collect (Harvest::unpack, engine/src/gpu/device.rs:759-831): wait for the
// wave, then split its outputs back into per-job, solve-local results.
bool Executor::collect(InFlight* f, std::vector<Result>* out, std::string* err) {
    if (!f->live) {
        *err = "nothing in flight to collect";
        return false;
    }
    Slot& sl = slots_[f->slot];
    f->live = false;
    sl.busy = false;
    in_flight_--;
    HIP_TRY(hipSetDevice(device_));
    HIP_TRY(hipEventSynchronize(sl.done));
    HIP_TRY(hipGetLastError());
    const float* strat = (const float*)sl.res;
    const float* roots = (const float*)(sl.res + f->o_roots);
    const uint16_t* carry = (const uint16_t*)(sl.res + f->o_carry);
    out->clear();
    uint32_t cell0 = 0, cfg0 = 0;
    for (const JobSlice& j : f->jobs) {
        Result r;
        r.weight_version = f->version;
        r.strategy.assign(strat + cell0, strat + cell0 + j.ncells);
        r.nroots = j.nroots;
        r.n0 = j.n0;
        r.n1 = j.n1;
        r.root_values.assign(roots + j.root_value0, roots + j.root_value0 + j.nroots * (j.n0 + j.n1));
        r.slots = (uint32_t)f->carry_slots;
        r.snapshot_configs = j.snapshot_configs;
        r.carries.resize(size_t(r.slots) * r.snapshot_configs);
        for (uint32_t s = 0; s < r.slots; s++)
            std::memcpy(r.carries.data() + size_t(s) * r.snapshot_configs,
                        carry + size_t(s) * f->snapshot_configs + cfg0, size_t(r.snapshot_configs) * 2);
        cell0 += j.ncells;
        cfg0 += r.snapshot_configs;
        out->push_back(std::move(r));
    }
    return true;
}

bool Executor::solve(const WaveHost& w, uint64_t version, std::vector<Result>* out, std::string* err) {
    InFlight f;
    if (!launch(w, version, &f, err)) return false;
    return collect(&f, out, err);
}

bool Executor::read_leaves(const WaveHost& w, const NetBank& bank, int p, std::vector<float>* values,
                           std::vector<float>* mass, std::string* err) {
    const size_t nout = readout_net(bank.ns.kind) ? w.tower_len : size_t(w.rows()) * bank.ns.heads;
    std::vector<float> head(nout);
    const size_t m0 = mass->size();
    mass->resize(m0 + size_t(w.rows()) * 2, 0.0f);
    if (nout) HIP_TRY(hipMemcpyAsync(head.data(), head_out_, nout * 4, hipMemcpyDeviceToHost, stream_));
    if (w.rows()) HIP_TRY(hipMemcpyAsync(mass->data() + m0, dev_.mass, size_t(w.rows()) * 2 * 4, hipMemcpyDeviceToHost,
                                         stream_));
    HIP_TRY(hipStreamSynchronize(stream_));
    // Each network-leaf value slot's net value, by the records the sweep reads.
    std::unordered_map<uint32_t, uint32_t> head_of;
    head_of.reserve(w.leaf_rec[p].size());
    for (const LeafRec& q : w.leaf_rec[p]) head_of[q.out] = q.head;
    for (uint32_t r = 0; r < w.rows(); r++) {
        const uint32_t node = w.row_node[r], base = w.vals_base[2 * node + p];
        for (uint32_t c = 0; c < w.nc(node, p); c++) {
            auto it = head_of.find(base + c);
            if (it == head_of.end() || it->second >= nout) {
                *err = "network row " + std::to_string(r) + " has a value slot without a leaf record";
                return false;
            }
            values->push_back(head[it->second]);
        }
    }
    return true;
}

bool Executor::leaf_probe(const WaveHost& w, uint64_t version, int traverser, std::vector<float>* values,
                          std::vector<float>* mass, std::string* err) {
    const NetBank* bank = bank_of(version, err);
    if (!bank) return false;
    if (traverser < 0 || traverser > 1) {
        *err = "the traverser must be 0 or 1";
        return false;
    }
    if (in_flight_) {
        *err = "collect the launched waves before probing";
        return false;
    }
    if (!upload(w, *bank, 0, err)) return false;
    if (bank->ns.kind == MODEL_TWO_TOWER) run_tower_private(*bank);
    if (bank->ns.kind == MODEL_V5) run_v5_build(*bank);
    static_products(*bank);
    init_state(w);
    leaf_net(*bank, traverser);
    HIP_TRY(hipGetLastError());
    values->clear();
    mass->clear();
    return read_leaves(w, *bank, traverser, values, mass, err);
}

bool Executor::leaf_trace(const WaveHost& w, uint64_t version, const std::vector<int32_t>& points, bool with_reach,
                          LeafTrace* out, std::string* err) {
    const NetBank* bank = bank_of(version, err);
    if (!bank) return false;
    if (in_flight_) {
        *err = "collect the launched waves before tracing";
        return false;
    }
    const int32_t iters = (int32_t)w.meta.iters, roots = (int32_t)w.nroots_max;
    // Output offsets of each requested point (values depend on its traverser).
    size_t nval[2] = {0, 0}, nreach = 0;
    for (uint32_t r = 0; r < w.rows(); r++) {
        const uint32_t node = w.row_node[r];
        nval[0] += w.nc(node, 0);
        nval[1] += w.nc(node, 1);
        nreach += size_t(w.nc(node, 0)) + w.nc(node, 1);
    }
    const size_t nmass = size_t(w.rows()) * 2;
    std::vector<size_t> voff(points.size());
    std::vector<int> seen(points.size(), 0);
    size_t vtot = 0;
    for (size_t k = 0; k < points.size(); k++) {
        const int32_t pt = points[k];
        if (pt >= iters || (pt < 0 && -pt > 2 * roots)) {
            *err = "trace point " + std::to_string(pt) + " is outside the schedule (" + std::to_string(iters) +
                   " iterations, " + std::to_string(roots) + " carried roots)";
            return false;
        }
        voff[k] = vtot;
        vtot += nval[pt >= 0 ? (pt & 1) : ((-pt - 1) & 1)];
    }
    out->values.assign(vtot, 0.0f);
    out->mass.assign(points.size() * nmass, 0.0f);
    out->reach.assign(with_reach ? points.size() * nreach : 0, 0.0f);
    if (!upload(w, *bank, 0, err)) return false;
    std::vector<float> reach(with_reach ? w.reach_len : 0), v, m;
    std::string herr;
    const LeafHook hook = [&](int32_t point, int p) {
        for (size_t k = 0; k < points.size(); k++) {
            if (points[k] != point || !herr.empty()) continue;
            v.clear();
            m.clear();
            std::string e;
            if (!read_leaves(w, *bank, p, &v, &m, &e)) {
                herr = e;
                return;
            }
            std::copy(v.begin(), v.end(), out->values.begin() + voff[k]);
            std::copy(m.begin(), m.end(), out->mass.begin() + k * nmass);
            seen[k] = 1;
            if (!with_reach) continue;
            if (w.reach_len &&
                hipMemcpy(reach.data(), dev_.reach, size_t(w.reach_len) * 4, hipMemcpyDeviceToHost) != hipSuccess) {
                herr = "hipMemcpy of the reach failed";
                return;
            }
            float* rr = out->reach.data() + k * nreach;
            for (uint32_t r = 0; r < w.rows(); r++) {
                const uint32_t node = w.row_node[r];
                for (int q = 0; q < 2; q++) {
                    const uint32_t b = w.reach_base[2 * node + q];
                    for (uint32_t c = 0; c < w.nc(node, q); c++) *rr++ = reach[b + c];
                }
            }
        }
    };
    run_schedule(w, *bank, nullptr, &hook);
    HIP_TRY(hipStreamSynchronize(stream_));
    HIP_TRY(hipGetLastError());
    if (!herr.empty()) {
        *err = herr;
        return false;
    }
    for (size_t k = 0; k < points.size(); k++)
        if (!seen[k]) {
            *err = "trace point " + std::to_string(points[k]) + " was not reached by the schedule";
            return false;
        }
    return true;
}

bool Executor::time_wave(const WaveHost& w, uint64_t version, uint32_t warmup, uint32_t reps, double* wave_ms,
                         ScheduleTimes* prof, std::string* err) {
    auto it = banks_.find(version);
    if (it == banks_.end()) {
        *err = "GPU weight version " + std::to_string(version) + " is unavailable";
        return false;
    }
    if (in_flight_) {
        *err = "collect the launched waves before timing";
        return false;
    }
    if (!upload(w, it->second, 0, err)) return false;
    hipGraphExec_t exec = nullptr;
    double build_ms = 0.0;
    if (graph_) {
        HIP_TRY(hipStreamSynchronize(stream_));
        if (!capture(w, it->second, &exec, &build_ms, err)) return false;
    }
    auto once = [&]() -> hipError_t {
        if (exec) return hipGraphLaunch(exec, stream_);
        run_schedule(w, it->second, nullptr);
        return hipSuccess;
    };
    for (uint32_t r = 0; r < warmup; r++) HIP_TRY(once());
    HIP_TRY(hipStreamSynchronize(stream_));
    HIP_TRY(hipGetLastError());
    hipEvent_t a, b;
    HIP_TRY(hipEventCreate(&a));
    HIP_TRY(hipEventCreate(&b));
    HIP_TRY(hipEventRecord(a, stream_));
    for (uint32_t r = 0; r < reps; r++) HIP_TRY(once());
    HIP_TRY(hipEventRecord(b, stream_));
    HIP_TRY(hipEventSynchronize(b));
    float ms = 0.0f;
    HIP_TRY(hipEventElapsedTime(&ms, a, b));
    hipEventDestroy(a);
    hipEventDestroy(b);
    if (exec) HIP_TRY(hipGraphExecDestroy(exec));
    *wave_ms = reps ? ms / reps : 0.0;
    if (prof) {
        run_schedule(w, it->second, prof);
        prof->graph_build_ms = build_ms;
    }
    HIP_TRY(hipGetLastError());
    return true;
}

bool Executor::mlp_forward(uint64_t version, uint32_t rows, const float* x, float* out, std::string* err) {
    auto it = banks_.find(version);
    if (it == banks_.end()) {
        *err = "GPU weight version unavailable";
        return false;
    }
    const NetShape& ns = it->second.ns;
    if (ns.kind != MODEL_MLP) {
        *err = "leaf-network inference alone takes the MLP; the two-tower net runs inside a wave";
        return false;
    }
    HIP_TRY(hipSetDevice(device_));
    const size_t esz = precision_ == WC_PRECISE || precision_ == WC_F16X ? 4 : 2;
    size_t mt = 0;
    auto mtake = [&](size_t bytes) {
        size_t a = align256(mt);
        mt = a + std::max<size_t>(bytes, 4);
        return a;
    };
    const size_t prow = precision_ == WC_PRECISE ? rows : gemm_rows(rows);  // GEMM operands: padded rows
    const std::vector<ChainPass> plan = plan_chain(nullptr, (rows + 15) / 16, ns.heads, cus_);
    if (!check_chain_plan(plan, nullptr, (rows + 15) / 16, ns.heads, err)) return false;
    size_t m_x = mtake(prow * ns.in * esz), m_h0 = mtake(prow * ns.hidden * esz), m_h1 = mtake(prow * ns.hidden * esz),
           m_out = mtake(size_t(rows) * ns.heads * 4), m_stage = mtake(size_t(rows) * ns.in * 4),
           m_plan = mtake(plan.size() * sizeof(ChainPass));
    if (!ensure(&mlp_, &mlp_cap_, mt, err)) return false;
    char* M = (char*)mlp_;
    X_ = M + m_x;
    H_[0] = M + m_h0;
    H_[1] = M + m_h1;
    S_[0] = S_[1] = nullptr;  // this layout holds no partial products
    head_out_ = (float*)(M + m_out);
    mlp_plan_ = (const ChainPass*)(M + m_plan);
    mlp_npass_ = (uint32_t)plan.size();
    if (!plan.empty())
        HIP_TRY(hipMemcpyAsync(M + m_plan, plan.data(), plan.size() * sizeof(ChainPass), hipMemcpyHostToDevice,
                               stream_));
    if (precision_ == WC_PRECISE) {
        HIP_TRY(hipMemcpyAsync(X_, x, size_t(rows) * ns.in * 4, hipMemcpyHostToDevice, stream_));
    } else {
        HIP_TRY(hipMemcpyAsync(M + m_stage, x, size_t(rows) * ns.in * 4, hipMemcpyHostToDevice, stream_));
        launch_to16(precision_, (const float*)(M + m_stage), X_, rows, ns.in, false, stream_);
    }
    run_mlp(it->second, rows, X_, nullptr, nullptr, mlp_plan_, mlp_npass_);
    HIP_TRY(hipGetLastError());
    HIP_TRY(hipMemcpyAsync(out, head_out_, size_t(rows) * ns.heads * 4, hipMemcpyDeviceToHost, stream_));
    HIP_TRY(hipStreamSynchronize(stream_));
    rows_ = 0;  // the wave buffers were repurposed; a later wave re-uploads
    return true;
}

bool Executor::time_mlp(uint64_t version, uint32_t rows, const float* x, uint32_t reps, double* chain_ms,
                        std::vector<double>* layer_ms, std::string* err) {
    auto it = banks_.find(version);
    if (it == banks_.end()) {
        *err = "GPU weight version unavailable";
        return false;
    }
    std::vector<float> tmp(size_t(rows) * it->second.ns.heads);
    if (!mlp_forward(version, rows, x, tmp.data(), err)) return false;  // uploads x, warms
    hipEvent_t a, b;
    HIP_TRY(hipEventCreate(&a));
    HIP_TRY(hipEventCreate(&b));
    HIP_TRY(hipEventRecord(a, stream_));
    for (uint32_t r = 0; r < reps; r++) run_mlp(it->second, rows, X_, nullptr, nullptr, mlp_plan_, mlp_npass_);
    HIP_TRY(hipEventRecord(b, stream_));
    HIP_TRY(hipEventSynchronize(b));
    float ms = 0.0f;
    HIP_TRY(hipEventElapsedTime(&ms, a, b));
    *chain_ms = reps ? ms / reps : 0.0;
    if (layer_ms) {
        std::vector<hipEvent_t> marks;
        hipEvent_t s0;
        HIP_TRY(hipEventCreate(&s0));
        HIP_TRY(hipEventRecord(s0, stream_));
        run_mlp(it->second, rows, X_, &marks, nullptr, mlp_plan_, mlp_npass_);
        HIP_TRY(hipStreamSynchronize(stream_));
        layer_ms->clear();
        hipEvent_t prev = s0;
        for (auto e : marks) {
            float lm = 0.0f;
            hipEventElapsedTime(&lm, prev, e);
            layer_ms->push_back(lm);
            prev = e;
        }
        for (auto e : marks) hipEventDestroy(e);
        hipEventDestroy(s0);
    }
    hipEventDestroy(a);
    hipEventDestroy(b);
    HIP_TRY(hipGetLastError());
    return true;
}

}  // namespace wc
