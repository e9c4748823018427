/*
 * wc_wave.h — C ABI of the MI355X (gfx950) wave executor.
 *
 * The reference's wave executor is a Rust crate (engine/src/gpu/) whose
 * callers hold a `GpuClient` and submit `PackedJob`s. This ABI is what that
 * crate's FFI would bind instead: plain pointers and sizes, the job in its
 * WCJ8 bytes (docs/TREE.md; engine/src/serialize.rs:1052-1129), results as
 * pointer+length views. Every call returns 0 on success or a negative code;
 * wc_last_error() then names the failure (the reference returns
 * Result<_, String> at the same points).
 */
#ifndef WC_WAVE_H
#define WC_WAVE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WC_OK 0
#define WC_ERR_INVALID -1   /* malformed input (bytes, shapes, arguments) */
#define WC_ERR_DEVICE -2    /* HIP runtime failure */
#define WC_ERR_GONE -3      /* the service has shut down */
#define WC_ERR_UNSUPPORTED -4

/* Leaf-net arithmetic. PRECISE reproduces the CPU net's float32 loop order
 * exactly (the reference's oracle mode, engine/src/gpu/device.rs:375-402);
 * F16/BF16 run the MFMA GEMM chain with f32 accumulation (the reference's
 * fast mode, CUBLAS_COMPUTE_32F_FAST_16F). F16X (no counterpart in the
 * reference) is compensated f16: every operand is held as an f16 pair
 * hi + lo and every product as three f16 MFMAs (hi hi + hi lo + lo hi) with
 * f32 accumulation, near float32 accuracy on the f16 matrix cores; MLP only,
 * layer by layer. */
#define WC_PRECISE 0
#define WC_F16 1
#define WC_BF16 2
#define WC_F16X 3

/* Thread-local text of the last failure on this thread. */
const char* wc_last_error(void);

/* Network description: the flat `set_weights(dims, w, b, ln)` bank
 * (engine/src/gpu/client.rs:257-272). dims[0] names the family:
 *   [5]                                                         the reference's v5 network
 *   [101, in, hidden, layers, heads, pool]                      MLP
 *   [102, in, width, pub_layers, priv_in, priv_layers, pool]    two-tower
 * w: MLP = W_1 [in x hidden] row-major, W_2..W_L [hidden x hidden],
 *    W_head [heads x hidden]; b = b_1..b_L [hidden], b_head [heads].
 * v5: w, b and ln in the blob order of NetLayout::new (engine/src/net.rs:272-316),
 *    ln = the (gain, shift) pair of every LayerNorm in application order. */
typedef struct wc_net_desc {
    const uint32_t* dims;
    uint32_t ndims;
    const float* w;
    size_t nw;
    const float* b;
    size_t nb;
    const float* ln; /* v5 only; the synthetic families take NULL, 0 */
    size_t nln;
} wc_net_desc;

/* Float counts a family expects for w and b (net.rs:272-316 for v5). */
int wc_net_sizes(const uint32_t* dims, uint32_t ndims, size_t* nw, size_t* nb);
/* Float count a family expects for ln (0 for the synthetic families). */
int wc_net_norms(const uint32_t* dims, uint32_t ndims, size_t* nln);

/* ------------------------------------------------------------ service API
 * Replaces service::spawn / GpuClient / SolveHandle
 * (engine/src/gpu/service.rs:55-82, client.rs:196-313). */

typedef struct wc_service wc_service;
typedef struct wc_ticket wc_ticket;
typedef struct wc_result wc_result;

typedef struct wc_service_opts {
    uint32_t lanes;        /* executor lanes (streams) per device; reference WARCHEST_WAVE_LANES, default 2 */
    uint32_t wave_jobs;    /* max jobs per wave; reference WARCHEST_WAVE_JOBS, default 64 */
    uint32_t wave_rows;    /* max network rows per wave; reference WARCHEST_WAVE_ROWS, default 49152 */
    uint32_t window_us;    /* bucket-fill window, counted from the seed job's arrival; reference WARCHEST_WAVE_US, default 800 */
    uint32_t whale_lanes;  /* lanes that take exclusive-route jobs; reference WARCHEST_WAVE_WHALE_LANES,
                              default (0) 1, clamped to 1..lanes (service.rs:100) */
    uint32_t class_shift;  /* coarsens the cost classes; reference WARCHEST_WAVE_CLASS_SHIFT, 0..2 (service.rs:993) */
    uint64_t route_unit;   /* bytes per route-threshold unit: exclusive >= 4, card-exclusive >= 6 units of
                              reservation (serialize.rs:174-201); 0 = 1 GiB, the reference's thresholds */
} wc_service_opts;

/* service::spawn(device, dims, w, b, ln, precise): blocks until every lane is
 * ready; fails if any lane fails (service.rs:55-82,144-162). opts may be NULL. */
int wc_service_create(int device, const wc_net_desc* net, int precision, const wc_service_opts* opts,
                      wc_service** out);
/* Drop of the last GpuClient: shuts the dispatcher down and joins (client.rs:293-300). */
void wc_service_destroy(wc_service* svc);
/* GpuClient::set_weights: returns the new monotone version (1, 2, ...; the bank given to
 * wc_service_create is version 0), or 0 on failure. Jobs already submitted keep the
 * version that was current when they were submitted (engine/src/gpu/service.rs:233). */
uint64_t wc_set_weights(wc_service* svc, const wc_net_desc* net);
/* GpuClient::queued_work: monotone cost estimate of queued and running work. */
uint64_t wc_queued_work(wc_service* svc);
/* GpuClient::submit_tagged: copies the job bytes; the ticket is completed when the wave finishes. */
int wc_submit(wc_service* svc, const uint8_t* job, size_t len, uint64_t tag, wc_ticket** out);
/* PreparedJob::new (client.rs:165-181): parse, validate and cost one WCJ8 job
 * once, for a service of `precision`. The handle is immutable and may be
 * submitted any number of times, from any thread, to any service of that
 * precision; each submission shares it (no copy, no re-parse). The job bytes
 * may be freed when this returns. */
typedef struct wc_prepared wc_prepared;
int wc_prepare(const uint8_t* job, size_t len, int precision, wc_prepared** out);
/* Its queued-work cost (client.rs:282-291). */
uint64_t wc_prepared_cost(const wc_prepared* p);
/* Drop the caller's handle; submissions still queued or running keep the job. */
void wc_prepared_free(wc_prepared* p);
/* GpuClient::submit_prepared / submit_tagged_prepared (client.rs:212-255). */
int wc_submit_prepared(wc_service* svc, const wc_prepared* job, uint64_t tag, wc_ticket** out);
/* SolveHandle::wait: blocks; *out owns the result (wc_result_free). Frees the ticket. */
int wc_wait(wc_ticket* t, wc_result** out);
/* 1 when wc_wait would not block, 0 otherwise. */
int wc_poll(const wc_ticket* t);
/* Drop a ticket without waiting for its result (the reference drops the
 * SolveHandle's receiver; the solve still runs and its result is discarded). */
void wc_ticket_free(wc_ticket* t);
/* Waves launched and guarded routes taken by the service so far (tooling). */
int wc_service_stats(wc_service* svc, uint64_t* waves, uint64_t* guarded_routes);

/* PackedJob::work and the service's view of one job (serialize.rs:159-201,394-431;
 * client.rs:282-291; service.rs:967-991), for admission, routing and tests:
 * the work vector as an executor of `precision` would run the job, its queued-work
 * cost and its cost class (route thresholds in units of route_unit bytes; 0 = 1 GiB). */
typedef struct wc_work_vector {
    uint64_t network_rows, legal_cells, reach_slots, reverse_nonzeros;
    uint64_t table_bytes, mutable_bytes, carried_output_bytes, levels;
    uint64_t reserved_bytes;
    uint32_t exclusive_route, arena_guard_route, card_exclusive_route; /* 0 / 1 */
} wc_work_vector;
int wc_job_work(const uint8_t* job, size_t len, int precision, uint64_t route_unit, uint32_t class_shift,
                wc_work_vector* out, uint64_t* cost, uint32_t* cost_class);

/* SolveResult views (client.rs:113-122). All indices are solve-local. */
uint64_t wc_result_tag(const wc_result* r);
uint64_t wc_result_weight_version(const wc_result* r);
/* Final average strategy, one float per legal cell (soff-aligned). */
const float* wc_result_strategy(const wc_result* r, size_t* n);
/* Root values: nroots x (n0 + n1) floats, player 0's configs first. */
const float* wc_result_root_values(const wc_result* r, uint32_t* nroots, uint32_t* n0, uint32_t* n1);
/* Carried beliefs, f16 bits: slots x snapshot_configs, laid out by the job's snap_coff. */
const uint16_t* wc_result_carries(const wc_result* r, uint32_t* slots, uint32_t* snapshot_configs);
/* SolveResult::{oversize_route, card_exclusive_route} (client.rs:120-121): the
 * routes the service took for the job (exclusive one-job wave; whole-device drain). */
int wc_result_routes(const wc_result* r, int* oversize_route, int* card_exclusive_route);
void wc_result_free(wc_result* r);

/* ------------------------------------------------------ executor (lane) API
 * Replaces Executor::{new, publish, launch, collect, solve}, Wave::pack and
 * Harvest::unpack (engine/src/gpu/device.rs:515-831, wave.rs:127-221): one
 * device; schedules in order on one stream, each wave's tables uploaded on a
 * second stream while the wave before it runs. */

typedef struct wc_executor wc_executor;
typedef struct wc_wave wc_wave;

int wc_executor_create(int device, int precision, wc_executor** out);
void wc_executor_destroy(wc_executor* ex);
/* Executor::publish: an immutable weight bank; returns its version (> 0) or 0 on failure. */
uint64_t wc_executor_publish(wc_executor* ex, const wc_net_desc* net);
/* Wave::pack: concatenate compatible jobs into one wave-global index space. */
int wc_wave_pack(const uint8_t* const* jobs, const size_t* lens, uint32_t njobs, wc_wave** out);
/* Packs new jobs into an existing wave, reusing its host buffers (no
 * counterpart in the reference, whose Wave::pack always builds a new wave:
 * for callers of wc_launch that pack wave after wave, as the service's lanes
 * do). A wave already launched may be repacked at once: wc_launch keeps what
 * the collection needs. If the jobs do not parse, the wave keeps its jobs; if
 * packing fails after that, the wave holds no jobs until it is repacked, and
 * every entry point taking it fails with WC_ERR_INVALID. */
int wc_wave_repack(wc_wave* w, const uint8_t* const* jobs, const size_t* lens, uint32_t njobs);
/* A 64-bit digest of every list and count of a packed wave, for tests and
 * tooling that compare two packings of the same jobs (no counterpart in the
 * reference). */
int wc_wave_digest(const wc_wave* w, uint64_t* out);
void wc_wave_free(wc_wave* w);

/* Counts of a packed wave, for admission, benchmarks and the roofline. */
typedef struct wc_wave_stats {
    uint32_t jobs, nodes, decision_nodes, chance_nodes, leaves, rows, terminals;
    uint32_t levels, iters, nroots_max, carry_slots;
    uint32_t units, top_levels;    /* subtree units, and the depths of the top regions swept per launch */
    uint32_t max_window;           /* value slots of the widest unit window (the sweep stages it in LDS) */
    uint64_t cells, reach_slots, reach_len, vals_len, rev_nnz, rvd_nnz, draw_nnz, snapshot_configs;
    uint64_t table_bytes, arena_bytes; /* device bytes: the uploaded immutable tables; the solve state */
    uint64_t cfr_bytes_per_iter[2]; /* algorithmic HBM bytes of one CFR iteration, traverser 0 / 1 */
    /* the same bytes by launch, [traverser][k]: subtree value sweep, top-region launches, subtree reach sweep,
     * average-strategy accumulation (run in the leaf-input launch) */
    uint64_t cfr_bytes_by_kernel[2][4];
    uint64_t mlp_flops_per_query;   /* trunk + every head row */
    /* one leaf-net pass over all network rows: FLOP the head-width-trimmed GEMMs
     * execute, and the algorithmic FLOP (trunk + the traverser's configs' head rows) */
    uint64_t mlp_flops_executed, mlp_flops_algorithmic;
    /* one leaf-input pooling of player p's network rows, 16-bit query inputs:
     * each row's reach and outputs, each distinct config list and embedding once */
    uint64_t leaf_input_bytes[2];
} wc_wave_stats;
int wc_wave_stats_get(const wc_wave* w, wc_wave_stats* out);

/* Read-only view of one packed table of a wave as uint32 words, by name, for
 * tests and tooling: the index lists "row_node", "reach_base", "vals_base",
 * "exit_node", "exit_coff", "legal_value", "child_start", "child",
 * "legal_off", "node_meta", "node_nc", "row_cfg", "row_cfg_off", "draw_to",
 * "rev_src", "rvd_src", "term_node", "unit_term"; the unit records "units"
 * (24 words each) and "trees" (12 words each); and per player p (0 or 1)
 * "back_rec<p>", "top_back_rec<p>", "reach_rec<p>", "top_reach_rec<p>",
 * "acc_rec<p>", "leaf_rec<p>" (4 words per record), "pool_grp<p>" (36 words
 * per group), "child_vb<p>", "back_lvl<p>", "reach_lvl<p>", the top regions'
 * rows "top_back<p>", "top_reach<p>" (node, config: 2 words each) and their
 * depth bounds "top_back_lvl<p>", "top_reach_lvl<p>", the top regions' value
 * launches "top_back_run<p>" (4 words each: depth, the second depth of a fused
 * pair or 0xFFFFFFFF, its first chunk bound, its chunk count) and their chunk
 * bounds "top_back_chunk<p>" (per fused pair, chunks + 1 row bounds in the
 * deeper depth, then chunks + 1 in the shallower), the reach pass's launches
 * "top_reach_run<p>" (4 words each, top-down: depth, the deeper depth of a
 * fused pair or 0xFFFFFFFF, its first chunk bound, its chunk count), their
 * chunk bounds "top_reach_chunk<p>" (per fused pair, chunks + 1 row bounds in
 * the deeper depth, then chunks + 1 bounds into "top_reach_par<p>", the
 * shallower rows each chunk computes), and "head_rb_n<p>" (the
 * head columns each 16-row block of network rows needs for traverser p). Returns NULL (and sets wc_last_error) for an unknown name;
 * *n receives the word count. The view lives as long as the wave. */
const uint32_t* wc_wave_array(const wc_wave* w, const char* name, size_t* n);

/* Test support (no counterpart in the reference): overwrite word `index` of
 * the packed table `name` (the names of wc_wave_array), for tests of the
 * bounds checks against a wave the packer did not make. The wave then counts
 * as unchecked: every later upload of it checks it on the device first. */
int wc_wave_poke(wc_wave* w, const char* name, size_t index, uint32_t value);

/* Checks every index of a packed wave that the device kernels follow (no
 * counterpart in the reference, whose kernels bound-check as they go). With ex
 * NULL, on the host: the check wc_wave_pack runs. With an executor, the check
 * an upload runs for a wave packed without it (a service wave of jobs
 * validated at submit): the structural checks on the host, then the element
 * tables uploaded to ex's device and checked there, nothing else launched;
 * `version` is a weight bank published on ex. WC_OK, or WC_ERR_INVALID with
 * "wave bounds: <the first failing condition>" in wc_last_error. */
int wc_wave_check(const wc_wave* w, wc_executor* ex, uint64_t version);

/* The fused value net's pass plan, for tests and tooling (no counterpart in
 * the reference, whose head GEMMs take fixed tiles: device.rs:1218-1305): for
 * nrb 16-row blocks whose head widths are cols[rb] (cols NULL: every block
 * needs `heads`) on a device of `cus` compute units, the passes in launch
 * order as rows of 10 uint32: block count n, head columns, then the n block
 * indices (the rest 0). Writes at most cap rows to out; *npass receives the
 * number of passes. */
int wc_value_net_plan(const uint32_t* cols, uint32_t nrb, uint32_t heads, uint32_t cus, uint32_t* out, size_t cap,
                      size_t* npass);

/* Executor::launch + collect (+ Harvest::unpack): runs the whole schedule,
 * blocks, and returns one result per job in submission order
 * (results[k] owned by the caller). */
int wc_solve_wave(wc_executor* ex, wc_wave* w, uint64_t version, wc_result** results);

/* Executor::launch (device.rs:596-757): queue the wave's upload, its whole
 * schedule and the result copies on the executor's stream and return at once.
 * The wave may be freed or repacked as soon as this returns. At most two waves
 * may be launched on one executor and not yet collected. */
typedef struct wc_inflight wc_inflight;
int wc_launch(wc_executor* ex, wc_wave* w, uint64_t version, wc_inflight** out);
/* 1 when wc_collect would not block, 0 otherwise. */
int wc_inflight_ready(const wc_executor* ex, const wc_inflight* f);
/* Executor::collect + Harvest::unpack (device.rs:759-831): wait, then one result
 * per job of the launched wave (results[k] owned by the caller). Frees f. */
int wc_collect(wc_executor* ex, wc_inflight* f, wc_result** results);

/* Tooling (no counterpart in the reference): the leaf net's values at the
 * initial reach (uniform strategy, root beliefs) for one traverser, computed
 * by the wave's own leaf-input and value-net kernels. values: for each network
 * row in wave order, the value of each of the row's configs of the traverser,
 * in the row's config order (*count receives the total; nothing is written
 * when it exceeds cap); mass (rows x 2, may be NULL): the rows' reach masses. */
int wc_wave_leaf_probe(wc_executor* ex, wc_wave* w, uint64_t version, int traverser, float* values, size_t cap,
                       size_t* count, float* mass);

/* Tooling (no counterpart in the reference): the same values captured inside
 * one whole schedule, right after the leaf net runs at each of `points`, so
 * the leaf-input and value-net kernels are checked at the reach the solve
 * itself produces. A point t >= 0 is iteration t (traverser t & 1); a point
 * -(1 + 2 r + p) is Phase 2's evaluation for carried root r and player p.
 * counts (4 entries) receives: [0] / [1] the values of one point of traverser
 * 0 / 1 (each network row's configs of that player, wave order), [2] the
 * network rows, [3] the reach floats of one point (each row's reach over its
 * configs, player 0's then player 1's). Outputs are concatenated over the
 * points in the order given: values (the sum of the points' value counts),
 * mass (2 * rows per point: the rows' reach masses), reach (counts[3] per
 * point; reach NULL: not captured). With values or mass NULL, or a buffer too
 * small, only counts is written. */
int wc_wave_leaf_trace(wc_executor* ex, wc_wave* w, uint64_t version, const int32_t* points, size_t npoints,
                       float* values, size_t values_cap, float* mass, size_t mass_cap, float* reach, size_t reach_cap,
                       size_t* counts);

/* Benchmark helper: upload once, run the full schedule `warmup` times
 * untimed, then `reps` times timed (inputs resident in HBM), returning the
 * mean device time per wave in milliseconds, measured with HIP events on the
 * executor's stream. kernel_ms (optional, 11 doubles) receives one profiled
 * schedule's device time per launch class: [0] CFR sweeps, [1] leaf net (all
 * of it, [9] and [10] included),
 * [2] leaf input, [3] everything else; [4] the mean device time of one CFR
 * iteration (all its sweep kernels), and the mean device time per iteration of
 * [5] the subtree value sweep, [6] the top-region launches (values and reach,
 * one launch per depth each), [7] the subtree reach sweep; [8] the host time
 * to capture and instantiate the schedule as one HIP graph (0 when the
 * executor runs without graphs: the environment variable WC_GRAPH=1 at
 * executor creation turns them on); [9] the leaf net's per-wave work (the v5
 * network's cards, trunk and config encoder; the two-tower net's private
 * tower; the MLP's fixed-column products); [10] the v5 network's joins over
 * the schedule (0 for the other nets). */
int wc_time_wave(wc_executor* ex, wc_wave* w, uint64_t version, uint32_t warmup, uint32_t reps, double* wave_ms,
                 double* kernel_ms);

/* Measurement helper (no counterpart in the reference): what this device
 * sustains, timed with HIP events. copy_gbs: a 16-byte nontemporal load/store
 * copy over two buffers of `bytes` (read + write traffic per second);
 * read_gbs: the same loads alone; mfma_tflops: v_mfma_f32_32x32x16_f16 on
 * register operands (f16 dense); mfma16_tflops: the same for
 * v_mfma_f32_16x16x32_f16, the instruction the fused value net issues.
 * Allocates 2 x bytes of device memory for the call. */
int wc_peak_probe(int device, size_t bytes, double* copy_gbs, double* read_gbs, double* mfma_tflops,
                  double* mfma16_tflops);

/* Leaf-net inference alone (the value-net GEMM chain): x is rows x in f32 on
 * the host; out receives rows x heads f32 (head rows 0..heads-1). */
int wc_mlp_forward(wc_executor* ex, uint64_t version, uint32_t rows, const float* x, float* out);
/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). wc_mlp_forward on device-resident buffers -- x: rows x in
 * f32, out: rows x heads f32 -- with every intermediate (the 16-bit input
 * operand, hidden activations, the pass plan) in one fixed device array of
 * WC_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends; the call
 * makes no device allocation. stream NULL: queued on the executor's stream
 * and the call waits for the result; otherwise queued on that hipStream_t and
 * the call returns at once. Calls that overlap on one GPU share the array and
 * race. Fails (WC_ERR_INVALID) when the rows need more than the array holds
 * (about 32k rows of a 512-input 16-bit net, 8k of the float32 net). */
#define WC_NOALLOC_SCRATCH_BYTES (32u << 20)
int wc_mlp_forward_noalloc(wc_executor* ex, uint64_t version, uint32_t rows, const float* x, float* out,
                           void* stream);
/* Benchmark helper for the chain alone: x resident on the device, `reps` launches,
 * mean milliseconds per chain from HIP events on the executor's stream. */
int wc_time_mlp(wc_executor* ex, uint64_t version, uint32_t rows, const float* x, uint32_t reps,
                double* chain_ms, double* layer_ms);

/* ------------------------------------------------- job contract utilities */

/* Decode and re-encode a WCJ8 job (byte-identical round trip), writing up to
 * cap bytes into out and the full length into *len. */
int wc_job_roundtrip(const uint8_t* job, size_t len, uint8_t* out, size_t cap, size_t* out_len);
/* Structural validation of one job (indices in range, CSRs monotone,
 * parents before children). */
int wc_job_validate(const uint8_t* job, size_t len);

/* Synthetic workloads (seeded). Trees grow breadth-first to a node budget,
 * decision nodes carry config-dependent legal cells grouped into public
 * observations, chance nodes carry per-config outcome rows, and every table
 * is packed the way engine/src/serialize.rs:689-956 packs a real solver. */
typedef struct wc_synth_spec {
    uint64_t seed;
    uint32_t trees;
    uint32_t nodes_lo, nodes_hi;
    uint32_t exact_decisions, exact_leaves;
    uint32_t act_lo, act_hi;
    float collapse;
    uint32_t chance;
    uint32_t draw_lo, draw_hi;
    uint32_t info_fixed;
    float info_median, info_p99;
    uint32_t info_cap;
    float legal_p, shift_p, notrans_p, terminal_p;
    uint32_t dirichlet;
    uint32_t nroots;
    float whale_frac;
    uint32_t whale_nodes, whale_info;
    uint32_t depth, iters, snapshots;
    float alpha, beta, gamma, predict;
    const uint32_t* net_dims;
    uint32_t n_net_dims;
} wc_synth_spec;

typedef struct wc_jobset wc_jobset;
void wc_synth_spec_default(wc_synth_spec* spec);
int wc_synth(const wc_synth_spec* spec, wc_jobset** out);
uint32_t wc_jobset_count(const wc_jobset* s);
const uint8_t* wc_jobset_job(const wc_jobset* s, uint32_t k, size_t* len);
void wc_jobset_free(wc_jobset* s);
/* Kaiming-normal weights and U[-0.1, 0.1] biases for a family (sizes from wc_net_sizes). */
int wc_synth_weights(const uint32_t* dims, uint32_t ndims, uint64_t seed, float* w, size_t nw, float* b,
                     size_t nb);
/* LayerNorm pairs for a family (v5: gains 1 + N(0, 0.01), shifts N(0, 0.01)). */
int wc_synth_norms(const uint32_t* dims, uint32_t ndims, uint64_t seed, float* ln, size_t nln);
/* rows x width features, U[0,1) with 30% of dims in one-hot blocks of width 8. */
int wc_synth_features(uint32_t rows, uint32_t width, uint64_t seed, float* x);

#ifdef __cplusplus
}
#endif

#endif /* WC_WAVE_H */
