// `kernelh tune` (GEMM autotune over precompiled gfx950 tile variants) and
// its per-candidate evaluator `kernelh tune-eval` (see tune.cpp).
#pragma once

namespace khcli {

// Orchestrator: never initialises HIP; evaluates each candidate in a child.
int run_tune(int argc, char **argv);

// One candidate in this process: re-verify, then time (prints a RESULT line).
int run_tune_eval(int argc, char **argv);

}  // namespace khcli
