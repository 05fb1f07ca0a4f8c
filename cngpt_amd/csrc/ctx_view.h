// ctx_view.h - what the training step (train_host.cpp) reads of a handle of
// cngpt_hip.cpp: its device, stream, shape and parameter views. Internal to
// the library (hidden symbols).
#pragma once
#include <hip/hip_runtime.h>

#include "../../include/cngpt_hip.h"
#include "kernels.h"

struct CtxView {
    int device;
    hipStream_t stream;
    cngpt_hip_config cfg;
    float* params;  // device, n_params floats in the weight-file layout
    long n_params;
    const float *wte, *wpe, *lnf_w, *lnf_b;
    const LayerW* layers;  // host array of n_layer views into params
};

// Fills v from h; -1 (message set) when h is null or holds no parameters.
__attribute__((visibility("hidden"))) int ctx_view(cngpt_hip_ctx* h, CtxView* v);
// Marks the packed weight copies stale after the parameters were updated
// in place (the next forward or decode entry point packs them again).
__attribute__((visibility("hidden"))) void ctx_params_written(cngpt_hip_ctx* h);
// Sets the message cngpt_hip_last_error() returns; returns -1.
__attribute__((visibility("hidden"))) int ctx_fail(const char* fmt, ...);
