// Element-wise chains with a kernel compiled for them (eltwise.hip's
// ew_chain_k instantiates one per entry, its steps as template arguments),
// shared by libnnc_hip.so and the cost-model runtime (host code only).
//
// A chain is nnc_hip_fused_eltwise's program: n_in inputs and n_steps steps
// {op, x, y} (NNC_EW_* op codes; an operand -1 is the previous step's value;
// a unary step's y is not used and is given as x). The table holds the
// chains the mi355x O3 compiler emits for its model set (the
// bandwidth-chain program's two) and a few common short ones.
#pragma once

#include "nnc_hip.h"

namespace nnc {

constexpr int kEwChainMaxSteps = 8;

struct EwChainDef {
    int n_in, n_steps;
    int prog[3 * kEwChainMaxSteps];
};

constexpr EwChainDef kEwChains[] = {
    // relu(x + y) * x, clip, sigmoid, + t
    {3, 5, {NNC_EW_ADD_RELU, 0, 1, NNC_EW_MUL, -1, 0, NNC_EW_CLIP, -1, -1, NNC_EW_SIGMOID, -1, -1, NNC_EW_ADD, -1, 2}},
    // tanh(x - y)
    {2, 2, {NNC_EW_SUB, 0, 1, NNC_EW_TANH, -1, -1}},
    // x * y + z
    {3, 2, {NNC_EW_MUL, 0, 1, NNC_EW_ADD, -1, 2}},
    // (x + y) * z
    {3, 2, {NNC_EW_ADD, 0, 1, NNC_EW_MUL, -1, 2}},
    // relu(x * y)
    {2, 2, {NNC_EW_MUL, 0, 1, NNC_EW_RELU, -1, -1}},
    // sigmoid(x + y) * y
    {2, 2, {NNC_EW_ADD_SIGMOID, 0, 1, NNC_EW_MUL, -1, 1}},
};
constexpr int kEwChainCount = (int)(sizeof kEwChains / sizeof kEwChains[0]);

// index into kEwChains of the chain (prog as nnc_hip_fused_eltwise takes
// it), or -1: same input count, steps, ops and operands (a unary step's y
// not compared)
inline int ew_chain_index(int n_in, const int* prog, int n_steps) {
    if (!prog) return -1;
    for (int c = 0; c < kEwChainCount; ++c) {
        const EwChainDef& d = kEwChains[c];
        if (d.n_in != n_in || d.n_steps != n_steps) continue;
        bool same = true;
        for (int s = 0; s < n_steps && same; ++s) {
            const int op = prog[3 * s];
            same = op == d.prog[3 * s] && prog[3 * s + 1] == d.prog[3 * s + 1] &&
                   (op > NNC_EW_ADD_SIGMOID || prog[3 * s + 2] == d.prog[3 * s + 2]);
        }
        if (same) return c;
    }
    return -1;
}

}  // namespace nnc
