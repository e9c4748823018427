// One device: weight banks, wave upload (on a copy stream, beside the schedule
// before it), the CFR schedule (on the executor's stream), results.
// Counterpart of the reference's `Executor` (engine/src/gpu/device.rs:515-831).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "job.h"
#include "kernels.h"
#include "v5.h"
#include "wave.h"

namespace wc {

struct NetBank {
    uint64_t version = 0;
    NetShape ns;
    int precision = 0;
    void* mem = nullptr;  // one device allocation holding every matrix and bias
    const void* W[16] = {};
    const float* B[16] = {};
    const void* Whead = nullptr;
    const float* bhead = nullptr;
    // Two-tower net: W/B hold the public tower; the private tower, the readout
    // weight (f32) and the readout bias.
    const void* PW[16] = {};
    const float* PB[16] = {};
    const float* wread = nullptr;
    float bread = 0.0f;
    // v5 network: the device view of its blob and board tables.
    v5::Net v5;
};

struct Result {
    uint64_t tag = 0;
    uint64_t weight_version = 0;
    bool oversize_route = false, card_exclusive_route = false;  // set by the service (client.rs:119-121)
    std::vector<float> strategy;
    uint32_t nroots = 0, n0 = 0, n1 = 0;
    std::vector<float> root_values;
    uint32_t slots = 0, snapshot_configs = 0;
    std::vector<uint16_t> carries;
};

// Per-launch-class device times of one schedule (milliseconds), from HIP events.
struct ScheduleTimes {
    double total = 0, cfr = 0, mlp = 0, leaf_input = 0, other = 0;
    double back_mean = 0, top_mean = 0, reach_mean = 0;  // mean duration of one launch of each CFR kernel
    double cfr_launch_mean = 0;  // mean device time of one CFR iteration (the three kernels)
    uint32_t cfr_launches = 0;
    double graph_build_ms = 0;   // host time to capture and instantiate the schedule's graph (0: not captured)
    double net_build = 0;        // the per-wave network work (v5 build, private tower, fixed-column products)
    double v5_join = 0;          // the v5 network's joins over the whole schedule (0 for other nets)
};

// Per-job facts the unpack of a collected wave needs, copied at launch so the
// packed wave can be reused (repacked) while the wave runs.
struct JobSlice {
    uint32_t ncells = 0, nroots = 0, n0 = 0, n1 = 0, root_value0 = 0, snapshot_configs = 0;
};

// One launched wave (the reference's `InFlight`, engine/src/gpu/device.rs:596-757):
// the schedule and the result copies are queued on the executor's stream; collect
// waits for them and splits the results per job.
struct InFlight {
    uint32_t slot = 0;
    uint64_t version = 0;
    std::vector<JobSlice> jobs;
    size_t ncells = 0, nroots = 0, carry_slots = 0, snapshot_configs = 0;
    size_t o_roots = 0, o_carry = 0;
    bool live = false;
};

// Leaf-net evaluations captured during a real schedule (Executor::leaf_trace),
// concatenated over the requested points in request order: per point the
// value of each network row's configs of that point's traverser (row order,
// row config order), the rows' reach masses [rows x 2], and each row's reach
// of both players over their configs (player 0's, then player 1's).
struct LeafTrace {
    std::vector<float> values, mass, reach;
};
// A schedule point: iteration t >= 0 (traverser t & 1), or Phase 2's
// evaluation for carried root r and player p as -(1 + 2 r + p).
constexpr int32_t phase2_point(uint32_t root, int p) { return -(1 + 2 * (int32_t)root + p); }

// The fused kernel's view of a 16-bit MLP bank.
ChainNet chain_net(const NetBank& bank);
// The allocation-free entry point's scratch array on `device` (current): its
// device address, looked up once per device (noalloc.hip).
bool noalloc_scratch(int device, void** out, std::string* err);

class Executor {
  public:
    Executor(int device, int precision);
    ~Executor();
    bool ok() const { return ok_; }
    const std::string& error() const { return err_; }
    int device() const { return device_; }
    int precision() const { return precision_; }
    hipStream_t stream() const { return stream_; }

    // Publish an immutable weight bank; returns its version (0 on failure).
    uint64_t publish(const NetShape& ns, const std::vector<uint32_t>& dims, const float* w, size_t nw,
                     const float* b, size_t nb, std::string* err, const float* ln = nullptr, size_t nln = 0);
    void retain_from(uint64_t oldest);
    bool has_version(uint64_t v) const { return banks_.count(v) != 0; }

    // Upload, run the whole schedule, collect one result per job.
    bool solve(const WaveHost& w, uint64_t version, std::vector<Result>* out, std::string* err);
    // Upload the wave and check its indices on the device (what an upload
    // runs for a wave that was not checked on the host), however it was packed.
    bool check(const WaveHost& w, uint64_t version, std::string* err);
    // The same in two halves: launch queues the upload, the schedule and the
    // result copies and returns; collect waits and unpacks. At most
    // MAX_IN_FLIGHT waves may be launched and not yet collected; the packed
    // wave may be reused as soon as launch returns. A wave checked on the
    // device makes launch wait for the check's result before it queues the
    // schedule; `meanwhile` (optional) is called once, while that check runs
    // (or once everything is queued), for a caller with other work such as
    // collecting its previous wave (it may call collect on this executor).
    static constexpr uint32_t MAX_IN_FLIGHT = 2;
    bool launch(const WaveHost& w, uint64_t version, InFlight* out, std::string* err,
                const std::function<void()>& meanwhile = {});
    bool collect(InFlight* f, std::vector<Result>* out, std::string* err);
    bool ready(const InFlight& f) const;
    uint32_t in_flight() const { return in_flight_; }
    // Executor::trim (engine/src/gpu/device.rs:574): release the grow-only device
    // buffers and pinned staging of past waves (the weight banks stay), so a
    // guarded wave on another lane finds the memory free. Fails while waves
    // are in flight.
    bool trim(std::string* err);
    // The leaf net's values at the initial reach (uniform strategy, root
    // beliefs) for one traverser, computed by the wave's own kernels: for each
    // network row in order, the value of each of the row's configs of the
    // traverser (row config order), and the reach masses [rows x 2].
    bool leaf_probe(const WaveHost& w, uint64_t version, int traverser, std::vector<float>* values,
                    std::vector<float>* mass, std::string* err);
    // The same values, masses and the reach that fed them, captured inside
    // one whole schedule right after the leaf net runs at each of `points`
    // (iterations and Phase 2 evaluations, phase2_point): the leaf-input and
    // value-net kernels at the reach the solve itself reaches.
    // with_reach false: the reach is not captured (out->reach stays empty).
    bool leaf_trace(const WaveHost& w, uint64_t version, const std::vector<int32_t>& points, bool with_reach,
                    LeafTrace* out, std::string* err);
    // Upload once, run `warmup` untimed schedules, then `reps` timed ones; mean
    // wave time, and per-class times of one extra profiled schedule.
    bool time_wave(const WaveHost& w, uint64_t version, uint32_t warmup, uint32_t reps, double* wave_ms,
                   ScheduleTimes* prof, std::string* err);
    // The leaf GEMM chain alone on rows x in host inputs.
    bool mlp_forward(uint64_t version, uint32_t rows, const float* x, float* out, std::string* err);
    // The same on device-resident x and out, every intermediate in the fixed
    // scratch array (no allocation); queued on `stream` (null: the executor's
    // stream, and waits).
    bool mlp_forward_noalloc(uint64_t version, uint32_t rows, const float* x, float* out, hipStream_t stream,
                             std::string* err);
    bool time_mlp(uint64_t version, uint32_t rows, const float* x, uint32_t reps, double* chain_ms,
                  std::vector<double>* layer_ms, std::string* err);

  private:
    // Copies the wave's tables into the pinned staging of `slot` and queues
    // their upload; sets up the device views of the wave.
    // A wave that did not pass validate_deep (`checked` false), or any wave
    // with device_check, is checked before the schedule may read it:
    // validate_shape on the host first, then the element tables on the device.
    bool launch_wave(const WaveHost& w, uint64_t version, InFlight* out, std::string* err,
                     std::function<void()>* meanwhile);
    // `meanwhile` (if set) is called and cleared while a device check runs.
    bool upload(const WaveHost& w, const NetBank& bank, uint32_t slot, std::string* err, bool device_check = false,
                std::function<void()>* meanwhile = nullptr);
    // The device element checks of the uploaded wave; waits for their result.
    bool check_on_device(const WaveHost& w, std::string* err, std::function<void()>* meanwhile);
    // hook (optional): called after every leaf-net evaluation with its
    // schedule point and traverser.
    using LeafHook = std::function<void(int32_t point, int p)>;
    void run_schedule(const WaveHost& w, const NetBank& bank, ScheduleTimes* prof, const LeafHook* hook = nullptr);
    // After a leaf-net evaluation for traverser p: copy the head outputs and
    // masses to the host and read each network row's config values of p by
    // the leaf records the sweep reads (appended to values and mass).
    bool read_leaves(const WaveHost& w, const NetBank& bank, int p, std::vector<float>* values,
                     std::vector<float>* mass, std::string* err);
    // Pieces of the schedule: the first layer's fixed-column products, the
    // initial CFR state (strategy, reach, sums, carries, leaf inputs), both
    // players' reach under a strategy, the top regions' value and reach
    // launches, one traverser's leaf net.
    void static_products(const NetBank& bank);
    void init_state(const WaveHost& w);
    void reach_both(const WaveHost& w, float* reach, const float* strat);
    void top_back(const WaveHost& w, int p, int mode, float da, float db, float pr);
    void top_reach(const WaveHost& w, int p, float* reach, const float* strat, float* reach2 = nullptr,
                   const float* strat2 = nullptr);
    void leaf_net(const NetBank& bank, int q);
    const NetBank* bank_of(uint64_t version, std::string* err) const;
    // The schedule captured into one HIP graph (kernels only: the schedule
    // issues no memset or copy) and instantiated; *build_ms gets the host time.
    bool capture(const WaveHost& w, const NetBank& bank, hipGraphExec_t* exec, double* build_ms, std::string* err);
    // Two-tower net: F for the uploaded wave's configs, then one traverser's public tower and readout.
    void run_tower_private(const NetBank& bank);
    void run_tower(const NetBank& bank, uint32_t rows, int traverser);
    // v5 network: publish its bank; the per-wave build (cards, trunk, configs)
    // for the uploaded wave under a bank, then per iteration the join and the readout.
    uint64_t publish_v5(const NetShape& ns, const float* w, size_t nw, const float* b, size_t nb, const float* ln,
                        size_t nln, std::string* err);
    void run_v5_build(const NetBank& bank);
    void run_v5(const NetBank& bank, int traverser);
    void run_v5_join(const NetBank& bank, int traverser);
    void run_v5_readout(const NetBank& bank, int traverser);
    // The MLP over `rows` query rows: the fused kernel over `plan` (npass
    // passes, device copy) where it applies, else layer by layer (head width
    // per 128-row tile: head_tile_n).
    // part: the first layer's precomputed product over the query inputs'
    // fixed columns (S_), or null.
    void run_mlp(const NetBank& bank, uint32_t rows, const void* x, std::vector<hipEvent_t>* marks,
                 const uint32_t* head_tile_n, const ChainPass* plan, uint32_t npass, const float* part = nullptr);
    bool ensure(void** p, size_t* cap, size_t need, std::string* err);
    bool ensure_pinned(uint8_t** p, size_t* cap, size_t need, std::string* err);

    int device_ = 0, precision_ = 0;
    uint32_t cus_ = 1;  // compute units of the device (fused value net plans)
    bool ok_ = false;
    std::string err_;
    hipStream_t stream_ = nullptr;
    hipStream_t copy_ = nullptr;  // table uploads and their device checks, beside the schedules
    std::map<uint64_t, NetBank> banks_;
    uint64_t next_version_ = 1;

    // Device buffers (grow-only): the immutable tables of each launch slot (a
    // wave's tables upload, and are checked, while the slot before it runs),
    // then the solve state and the value net's buffers the waves use in turn.
    void* table_[MAX_IN_FLIGHT] = {};
    size_t table_cap_[MAX_IN_FLIGHT] = {};
    void* arena_ = nullptr;
    size_t arena_cap_ = 0;
    void* mlp_ = nullptr;  // query inputs, hidden activations, head outputs
    size_t mlp_cap_ = 0;
    // Per launch slot: pinned staging of the table blob and pinned landing of
    // the collected outputs (grow-only), and events marking the end of the
    // slot's upload and of its wave.
    struct Slot {
        uint8_t* pin = nullptr;
        size_t pin_cap = 0;
        uint8_t* res = nullptr;
        size_t res_cap = 0;
        hipEvent_t uploaded = nullptr, done = nullptr;
        bool recorded = false;  // `uploaded` has been recorded at least once
        bool busy = false;      // launched, not yet collected
        hipGraphExec_t exec = nullptr;  // the launched wave's captured schedule
    };
    Slot slots_[MAX_IN_FLIGHT];
    uint32_t in_flight_ = 0;
    WaveDev dev_{};
    void* X_ = nullptr;
    void* Xq_[2] = {};  // the wave's query inputs, one per traverser
    uint32_t* check_ = nullptr;       // the device check's flag word and pool-group row counters (after the tables)
    uint32_t* check_host_ = nullptr;  // pinned landing of the flag word
    const BackRec* top_back_dev_[2] = {};    // top-region rows by depth (device copies)
    const ReachRec* top_reach_dev_[2] = {};
    const uint32_t* top_chunk_dev_[2] = {};  // chunk bounds of the fused value launches
    const uint32_t* top_reach_chunk_dev_[2] = {};  // chunk bounds of the fused reach launches
    const uint32_t* top_reach_par_dev_[2] = {};    // and the shallower rows each chunk computes
    const uint32_t* head_tile_n_ = nullptr;  // head width per 128-row tile (device copy)
    const ChainPass* chain_plan_[2] = {};    // fused value net passes per traverser (device copies)
    uint32_t chain_npass_[2] = {0, 0};
    const ChainPass* mlp_plan_ = nullptr;    // the same for mlp_forward's rows
    uint32_t mlp_npass_ = 0;
    void* H_[2] = {};
    // The fused value net's first-layer product over each traverser's fixed
    // query columns (seat, public features), f32 accumulator tiles; computed
    // at the start of each schedule (null where the fused net does not run).
    float* S_[2] = {};
    float* head_out_ = nullptr;  // MLP head outputs, or the two-tower readout per (row, config)
    // Two-tower net: private-tower input, layer outputs and F (one row per interned config).
    const float* cfg_priv_ = nullptr;
    void* PX_ = nullptr;
    void* P_[2] = {};
    void* F_ = nullptr;
    uint32_t ncfg_ = 0;
    uint32_t rows_ = 0;
    // v5 network: the uploaded wave's build inputs, its per-wave outputs and
    // the join's float32 input scratch (16-bit path).
    v5::WaveIn v5_in_{};
    v5::WaveOut v5_out_{};
    float* v5_xf_ = nullptr;
    void* scratch_ = nullptr;  // the allocation-free scratch on this device
    std::string scratch_err_;
    bool split_ = true;  // WC_CHAIN_SPLIT=0 turns the first layer's fixed-column product off
    bool graph_ = false; // WC_GRAPH=1: each wave's schedule runs as one captured HIP graph
    // WC_UNIT_LDS=0: the sweep and reach passes read and write unit windows in
    // HBM only (the paths taken when a window does not fit LDS)
    bool unit_lds_ = true;
    // WC_V5_SCALAR=1: the v5 network's 16-bit path without the matrix cores
    // (rounded operands, float32 sums in ascending order)
    bool v5_scalar_ = false;
};

}  // namespace wc
