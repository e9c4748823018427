// The allocation-free leaf-net entry point: wc_mlp_forward on device-resident
// inputs and outputs, every intermediate carved from one fixed device array.
//
// For callers that cannot call hipMalloc (code under HIP graph capture, tight
// serving loops, harnesses that forbid it). The array is a file-scope device
// variable: each GPU the library runs on holds its own copy, at its own
// address, until the process ends. Host code never passes the variable's name
// to a kernel (in host code it is a stand-in, not a device address): the
// device address comes from hipGetSymbolAddress, once per device, with that
// device current, and every kernel argument and copy uses that address.
// Every call on a GPU shares the array, which keeps the last call's contents;
// calls that overlap on one GPU race.
#include <algorithm>
#include <mutex>

#include "../../include/wc_wave.h"
#include "executor.h"
#include "kernels.h"

namespace wc {

static_assert(WC_NOALLOC_SCRATCH_BYTES % 256 == 0, "scratch is carved in 256-byte aligned pieces");
static __device__ __align__(256) uint8_t scratch[WC_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch[MAX_DEVICES] = {};  // the array's device address on each device

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// Passes of up to CHAIN_PASS_BLOCKS consecutive 16-row blocks, every pass
// computing all `cols` head columns: the plan of rows that all need the
// whole head, written on the device (no host buffer, no copy).
__global__ void k_plan_consecutive(ChainPass* plan, uint32_t nrb, uint32_t cols) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t npass = (nrb + CHAIN_PASS_BLOCKS - 1) / CHAIN_PASS_BLOCKS;
    if (i >= npass) return;
    ChainPass ps;
    ps.n = min(CHAIN_PASS_BLOCKS, nrb - i * CHAIN_PASS_BLOCKS);
    for (uint32_t j = 0; j < CHAIN_PASS_BLOCKS; j++) ps.rb[j] = j < ps.n ? i * CHAIN_PASS_BLOCKS + j : 0u;
    ps.cols = cols;
    ps.pad[0] = ps.pad[1] = 0;
    plan[i] = ps;
}

}  // namespace

// The scratch array's address on `device`, looked up the first time a device
// asks (the caller has made it current).
bool noalloc_scratch(int device, void** out, std::string* err) {
    if (device < 0 || device >= MAX_DEVICES) {
        *err = "device ordinal out of range for the allocation-free scratch";
        return false;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch[device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            *err = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
            return false;
        }
        g_scratch[device] = p;
    }
    *out = g_scratch[device];
    return true;
}

bool Executor::mlp_forward_noalloc(uint64_t version, uint32_t rows, const float* x, float* out, hipStream_t stream,
                                   std::string* err) {
    const NetBank* bank = bank_of(version, err);
    if (!bank) return false;
    const NetShape& ns = bank->ns;
    if (ns.kind != MODEL_MLP) {
        *err = "the allocation-free leaf-net entry point takes the MLP";
        return false;
    }
    if (!scratch_) {
        *err = scratch_err_.empty() ? "the allocation-free scratch is unavailable" : scratch_err_;
        return false;
    }
    if (rows == 0) return true;
    // The pieces of one call, 256-byte aligned: the pass plan (fused net), the
    // 16-bit input operand (rows padded to GEMM_ROWS; compensated f16: hi and
    // lo planes), the hidden activations (layer-by-layer nets).
    const bool fused = (precision_ == WC_F16 || precision_ == WC_BF16) && chain_fits(ns.in, ns.hidden, ns.layers);
    const size_t esz = precision_ == WC_F16X ? 4 : 2;
    const size_t prow = precision_ == WC_PRECISE ? rows : gemm_rows(rows);
    const uint32_t nrb = (rows + 15) / 16, npass = (nrb + CHAIN_PASS_BLOCKS - 1) / CHAIN_PASS_BLOCKS;
    size_t at = 0;
    auto take = [&](size_t bytes) {
        const size_t a = align256(at);
        at = a + bytes;
        return a;
    };
    const size_t o_plan = fused ? take(size_t(npass) * sizeof(ChainPass)) : 0;
    const size_t o_x = precision_ == WC_PRECISE ? 0 : take(prow * ns.in * esz);
    const size_t hbytes = prow * ns.hidden * (precision_ == WC_PRECISE ? 4 : esz);
    const size_t o_h0 = fused ? 0 : take(hbytes), o_h1 = fused ? 0 : take(hbytes);
    if (at > WC_NOALLOC_SCRATCH_BYTES) {
        const size_t per_row = std::max<size_t>(at / std::max<uint32_t>(rows, 1), 1);
        *err = std::to_string(rows) + " rows need " + std::to_string(at) + " bytes of scratch; the allocation-free "
               "entry point holds " + std::to_string(size_t(WC_NOALLOC_SCRATCH_BYTES)) + " (about " +
               std::to_string(WC_NOALLOC_SCRATCH_BYTES / per_row) + " rows of this network)";
        return false;
    }
    if (hipSetDevice(device_) != hipSuccess) {
        *err = "hipSetDevice failed";
        return false;
    }
    uint8_t* base = (uint8_t*)scratch_;
    hipStream_t s = stream ? stream : stream_;
    if (precision_ == WC_PRECISE) {
        const float* in = x;
        uint32_t k = ns.in;
        for (uint32_t l = 0; l < ns.layers; l++) {
            float* o = (float*)(base + (l & 1 ? o_h1 : o_h0));
            launch_dense_exact(in, k, (const float*)bank->W[l], bank->B[l], ns.hidden, o, rows, s);
            in = o;
            k = ns.hidden;
        }
        launch_head_exact(in, ns.hidden, (const float*)bank->Whead, bank->bhead, ns.heads, out, rows, s);
    } else {
        void* xop = base + o_x;
        launch_to16(precision_, x, xop, rows, ns.in, false, s);
        if (fused) {
            ChainPass* plan = (ChainPass*)(base + o_plan);
            hipLaunchKernelGGL(k_plan_consecutive, dim3((npass + 63) / 64), dim3(64), 0, s, plan, nrb, ns.heads);
            launch_chain(precision_, chain_net(*bank), xop, rows, out, plan, npass, s);
        } else {
            const void* in = xop;
            uint32_t k = ns.in;
            for (uint32_t l = 0; l < ns.layers; l++) {
                void* o = base + (l & 1 ? o_h1 : o_h0);
                launch_gemm16(precision_, in, k, bank->W[l], bank->B[l], ns.hidden, o, rows, true, true, s);
                in = o;
                k = ns.hidden;
            }
            launch_gemm16(precision_, in, ns.hidden, bank->Whead, bank->bhead, ns.heads, out, rows, false, false, s);
        }
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        *err = std::string("leaf-net launch: ") + hipGetErrorString(e);
        return false;
    }
    if (!stream && hipStreamSynchronize(s) != hipSuccess) {
        *err = "hipStreamSynchronize failed";
        return false;
    }
    return true;
}

}  // namespace wc
