// zi_sample.hip -- launchers of the sampling kernels (zi_sample_kernels.hpp):
// the instance for each (dtype, vectors per thread, mask, penalties) and the
// choice between the chunked kernels and one workgroup per row.
#include "zi_sample_kernels.hpp"

#ifndef ZI_SAMPLE_CAP
#define ZI_SAMPLE_CAP 0
#endif

namespace zi {

template <bool NUC, bool CAP, typename T, int NV, bool M, bool PN>
static hipError_t launch_sample_t(const SampleParams &P, int rows, hipStream_t st) {
    if (rows >= kRowLoopRows) {  // one workgroup per row fills the device
        // min_p > 0: the streamed prefix (zi_prefix.hpp), eight 16-byte
        // vectors per thread per step (four with a softcap or for masked bf16
        // rows, whose extra state would not fit the registers beside eight)
        constexpr int NVM = (CAP || (std::is_same<T, uint16_t>::value && M)) ? 4 : 8;
        if (NUC && P.min_p > 0.0f)
            hipLaunchKernelGGL((prefix_kernel<T, NVM, M, PN, CAP>), dim3(rows), dim3(kThreads), 0, st, P);
        else
            hipLaunchKernelGGL((row_kernel<T, NV, M, PN, NUC, CAP>), dim3(rows), dim3(kThreads), 0, st, P);
        return hipGetLastError();
    }
    dim3 grid(rows * P.src.G), block(kThreads);
    if constexpr (NUC) {
        hipLaunchKernelGGL((nucleus_kernel<T, NV, M, PN, CAP>), grid, block, 0, st, P);
    } else if constexpr (PN) {
        // Penalties that never raise a logit (edits are checked per chunk in
        // the kernel) take the late-penalty select when the grid is large
        // enough for the history to arrive behind other workgroups' rows
        // (config 1, 4 workgroups, measured 0.13 us faster with the
        // in-stream penalties; config 2, 256 workgroups, 0.72 us slower).
        const RowSource &a = P.src;
        // The late select relies on few raw candidates: once they overflow
        // the per-wave staging it selects again.  Measured on config-2 rows
        // (64 x 128256 f32, penalties), us per call, late against in-stream:
        // k = 32 15.9 / 16.6, k = 48 16.8 / 17.6, k = 58 17.4 / 18.1,
        // k = 60 18.3 / 18.8, k = 64 18.4 / 18.8 (k = 60 and 64 with the
        // bisection threshold), k = 100 37.1 / 24.0.
        const bool late = rows * a.G >= kLatePenMinGroups && P.k <= kLatePenMaxK && (!a.do_rep || a.rp >= 1.0f) &&
                          (!a.do_fp || (a.freq >= 0.0f && a.pres >= 0.0f));
        if (late) hipLaunchKernelGGL((sample_kernel<T, NV, M, PN, CAP, true>), grid, block, 0, st, P);
        else hipLaunchKernelGGL((sample_kernel<T, NV, M, PN, CAP, false>), grid, block, 0, st, P);
    } else {
        hipLaunchKernelGGL((sample_kernel<T, NV, M, PN, CAP, false>), grid, block, 0, st, P);
    }
    return hipGetLastError();
}

template <bool NUC, bool CAP, typename T, int NV>
static hipError_t launch_sample_nv(const SampleParams &P, int rows, hipStream_t st) {
    const bool m = P.src.mask != nullptr;
    const bool p = (P.src.hist != nullptr) || (P.src.edit_ids != nullptr);
    if (m && p) return launch_sample_t<NUC, CAP, T, NV, true, true>(P, rows, st);
    if (m) return launch_sample_t<NUC, CAP, T, NV, true, false>(P, rows, st);
    if (p) return launch_sample_t<NUC, CAP, T, NV, false, true>(P, rows, st);
    return launch_sample_t<NUC, CAP, T, NV, false, false>(P, rows, st);
}

template <bool NUC, bool CAP>
static hipError_t launch_dispatch(const SampleParams &P, int dtype, int nv, int rows, hipStream_t st) {
    if (dtype == 0) {
        switch (nv) {
            case 4: return launch_sample_nv<NUC, CAP, float, 4>(P, rows, st);
            case 8: return launch_sample_nv<NUC, CAP, float, 8>(P, rows, st);
            default: return launch_sample_nv<NUC, CAP, float, 16>(P, rows, st);
        }
    }
    switch (nv) {
        case 2: return launch_sample_nv<NUC, CAP, uint16_t, 2>(P, rows, st);
        case 4: return launch_sample_nv<NUC, CAP, uint16_t, 4>(P, rows, st);
        default: return launch_sample_nv<NUC, CAP, uint16_t, 8>(P, rows, st);
    }
}

// This file is compiled twice: as itself (the uncapped instances and the
// public launchers) and through zi_sample_cap.hip with ZI_SAMPLE_CAP = 1 (the
// softcap instances), so the two halves build in parallel.
#if ZI_SAMPLE_CAP
hipError_t launch_sample_capped(const SampleParams &P, int dtype, int nv, int rows, hipStream_t st) {
    return launch_dispatch<false, true>(P, dtype, nv, rows, st);
}

hipError_t launch_nucleus_capped(const SampleParams &P, int dtype, int nv, int rows, hipStream_t st) {
    return launch_dispatch<true, true>(P, dtype, nv, rows, st);
}
#else
hipError_t launch_sample(const SampleParams &P, int dtype, int nv, int rows, hipStream_t st) {
    if (P.src.cap > 0.0f) return launch_sample_capped(P, dtype, nv, rows, st);
    return launch_dispatch<false, false>(P, dtype, nv, rows, st);
}

hipError_t launch_nucleus(const SampleParams &P, int dtype, int nv, int rows, hipStream_t st) {
    if (P.src.cap > 0.0f) return launch_nucleus_capped(P, dtype, nv, rows, st);
    return launch_dispatch<true, false>(P, dtype, nv, rows, st);
}
#endif

}  // namespace zi
