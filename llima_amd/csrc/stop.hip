// stop.hip -- the decode loop's stop-token check on the device (gfx950).
//
// Restates the reference's per-step stop rule (sima-neat/llima, paths relative
// to that repository): a token in the stop set ends generation and is kept
// (plain decode sima_lmm/devkit/cpp/language_model.cpp:643-671, prefill token
// :437-440); a speculative step's emitted run is cut after its first stop token
// and at the room left in the cache (DFlash language_model_dflash.cpp:570-579,
// Gemma4 MTP language_model_gemma4_mtp.cpp:940-956).  The stop set is a
// bitmask over the vocabulary (bit id & 31 of word id >> 5, LSB first), so a
// lookup is one load; ids outside [0, V) never stop.  One thread per
// sequence: the work is a few loads and compares, and the result stays on the
// device, where the next step's launch reads it.
#include "common.hpp"
#include "../../include/llima_sampler.h"

namespace llima {

struct StopParams {
    const int32_t* tokens;   // [B][M]
    const int32_t* count;    // [B] or null (M)
    const int32_t* room;     // [B] or null (no cap)
    const uint32_t* stop;    // [ceil(V / 32)]
    int32_t* out_keep;       // [B]
    int32_t* out_status;     // [B] or null
    int32_t B, M, V;
};

__global__ __launch_bounds__(LLIMA_WG) void stop_check_kernel(StopParams P) {
    const int b = (int)(blockIdx.x * LLIMA_WG + threadIdx.x);
    if (b >= P.B) return;
    int n = P.count ? P.count[b] : P.M;
    n = n < 0 ? 0 : (n > P.M ? P.M : n);
    int cap = n, status = LLIMA_STOP_NONE;
    if (P.room) {
        // a run that reaches the room fills the cache, also when it fits
        // exactly (language_model_gemma4_mtp.cpp:953-955, 1011-1012;
        // language_model_dflash.cpp:625-626); a stop token inside it wins
        const int r = P.room[b] < 0 ? 0 : P.room[b];
        if (r <= n) { cap = r; status = LLIMA_STOP_CACHE_FULL; }
    }
    const int32_t* tk = P.tokens + (size_t)b * P.M;
    int keep = cap;
    for (int i = 0; i < cap; ++i) {
        const int32_t id = tk[i];
        const bool hit = id >= 0 && id < P.V && ((P.stop[id >> 5] >> (id & 31)) & 1u);
        if (hit) { keep = i + 1; status = LLIMA_STOP_TOKEN; break; }
    }
    P.out_keep[b] = keep;
    if (P.out_status) P.out_status[b] = status;
}

}  // namespace llima

using namespace llima;

extern "C" int llima_stop_check(const int32_t* tokens, const int32_t* count, int32_t B, int32_t M,
                                const uint32_t* stop_mask, int32_t V, const int32_t* room,
                                int32_t* out_keep, int32_t* out_status, void* stream) {
    if (B < 0 || M < 0 || V <= 0) return LLIMA_E_INVAL;
    if (B == 0) return LLIMA_OK;
    if ((M > 0 && !tokens) || !stop_mask || !out_keep) return LLIMA_E_INVAL;
    StopParams P;
    P.tokens = tokens; P.count = count; P.room = room; P.stop = stop_mask;
    P.out_keep = out_keep; P.out_status = out_status;
    P.B = B; P.M = M; P.V = V;
    const uint32_t g = (uint32_t)((B + LLIMA_WG - 1) / LLIMA_WG);
    hipLaunchKernelGGL(stop_check_kernel, dim3(g), dim3(LLIMA_WG), 0, (hipStream_t)stream, P);
    return hipGetLastError() == hipSuccess ? LLIMA_OK : LLIMA_E_HIP;
}
