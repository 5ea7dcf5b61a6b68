// mmh_gemm_noalloc: the GEMM seam (mmh_gemm_nn/nt/tn) for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc). The only device memory the GEMM needs
// beyond its operands is the split-K partials ([splits, m, n] f32, written in
// full by the splits and summed in split order by the last split of each
// tile) with one counter per tile, and the tail pieces of the 128x128 kernel
// (summed by tail_reduce); here they live in file-scope device arrays of
// fixed size instead of the context's growable workspace and counters, so no
// call allocates or frees anything.
//
// The arrays exist once per GPU (each device that loads this code object
// holds its own copy until the process ends). Their device addresses are
// looked up with hipGetSymbolAddress once per device, with that device
// current, and only those addresses are ever handed to kernels. Every call on
// one GPU shares them: calls that overlap on one GPU (two streams, two
// contexts, two threads) race on them. Nothing in them needs clearing between
// calls: each split or piece writes every element of its partial tile before
// it is summed, and the counters start at zero (the arrays are zero when the
// code object loads) and are reset by the split that completes a tile.
#include <mutex>

#include "mmh_internal.h"

namespace mmh {
namespace {

constexpr size_t kScratchBytes = size_t(16) << 20;  // 16 MiB per GPU: the benchmark sweep's largest partials

static __device__ __align__(256) float scratch[kScratchBytes / 4];
// The split-K tile counters (zero when the code object loads; the last split
// of a tile resets its counter, so they are zero between calls).
static __device__ __align__(256) int32_t scratch_tickets[Context::kTickets];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float *g_scratch_ptr[kMaxDevices] = {};
int32_t *g_tickets_ptr[kMaxDevices] = {};

// The device addresses of `scratch` and `scratch_tickets` on ctx's device
// (current: context() selects it), looked up on the first call on that device.
float *scratch_of(const Context &ctx, int32_t **tickets) {
    if (ctx.device < 0 || ctx.device >= kMaxDevices)
        fail(MMH_ERR_ARGUMENT, "gemm_noalloc: device index out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    float *&ptr = g_scratch_ptr[ctx.device];
    int32_t *&tk = g_tickets_ptr[ctx.device];
    if (!ptr || !tk) {
        void *addr = nullptr, *taddr = nullptr;
        check_hip(hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)), "gemm_noalloc scratch lookup");
        check_hip(hipGetSymbolAddress(&taddr, HIP_SYMBOL(scratch_tickets)),
                  "gemm_noalloc counter lookup");
        if (!addr || !taddr)
            fail(MMH_ERR_DEVICE, "gemm_noalloc: the scratch arrays have no device address");
        ptr = static_cast<float *>(addr);
        tk = static_cast<int32_t *>(taddr);
    }
    *tickets = tk;
    return ptr;
}

}  // namespace
}  // namespace mmh

using namespace mmh;

extern "C" {

int32_t mmh_gemm_noalloc(mmh_handle ctx, int32_t form, const float *a, const float *b,
                         float *c, int64_t m, int64_t k, int64_t n, int32_t accumulate) {
    return guard([&] {
        Context &cx = context(ctx);
        if (form != MMH_GEMM_NN && form != MMH_GEMM_NT && form != MMH_GEMM_TN)
            fail(MMH_ERR_ARGUMENT, "gemm_noalloc: form must be MMH_GEMM_NN, _NT or _TN, got " +
                                       std::to_string(form));
        if (!a || !b || !c) fail(MMH_ERR_ARGUMENT, "gemm_noalloc: a null operand pointer");
        if (m <= 0 || k <= 0 || n <= 0)
            fail(MMH_ERR_SHAPE, "gemm_noalloc: m, k and n must be at least 1");
        const bool ta = form == MMH_GEMM_TN, tb = form == MMH_GEMM_NT;
        GemmDesc d;
        d.a = a;
        d.b = b;
        d.c = c;
        d.m = m;
        d.k = k;
        d.n = n;
        d.ta = ta;
        d.tb = tb;
        d.lda = ta ? m : k;
        d.ldb = tb ? k : n;
        d.ldc = n;
        d.epi = accumulate ? EPI_ACCUM : EPI_STORE;
        d.accumulate_into_c = accumulate != 0;
        d.scratch = scratch_of(cx, &d.scratch_tickets);
        d.scratch_bytes = kScratchBytes;
        gemm(cx, d);
        return MMH_OK;
    });
}

}  // extern "C"
