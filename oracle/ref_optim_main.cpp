// ref_optim_main.cpp -- TEST INFRASTRUCTURE ONLY.
//
// Runner for the reference's own optimizer suite (tests/test_optimizer.cpp in
// the reference), compiled where it lies against this build's drop-in
// Tensor, optimizers, losses and modules (whitematter_amd/core/tensor.h,
// optimizer.h, loss.h, layer.h, force-included so that they stand in for the
// reference's headers).  Built by oracle/Makefile into
// oracle/_ref/run_ref_optim; run on the GPU by tests/test_gpu_ref_suites.py.
#include "test_framework.h"

TestSuite* create_optimizer_tests();

int main() {
    TestRunner runner;
    runner.add_suite(create_optimizer_tests());
    return runner.run_all();
}
