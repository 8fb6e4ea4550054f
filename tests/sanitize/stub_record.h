// What the stub launchers of the sanitizer build record (stub_launchers.cpp).
#pragma once

#include "fa_params.hpp"

struct StubRecord {
    fa::FwdParams fwd{};
    fa::BwdParams bwd{};
    fa::DbiasReduceParams reduce{};
    int D = 0, stage = 0;
    bool causal = false, dropout = false;
    int fwd_calls = 0, bwd_calls = 0, keep_bits_calls = 0, reduce_calls = 0, misc_calls = 0;
    const char* last = "";
};

extern StubRecord g_stub;
