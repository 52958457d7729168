// ref_loss_main.cpp -- TEST INFRASTRUCTURE ONLY.
//
// Runner for the reference's own loss suite (tests/test_loss.cpp in the
// reference), compiled where it lies against this build's drop-in Tensor and
// losses (whitematter_amd/core/tensor.h and loss.h, force-included so that
// they stand in for the reference's headers) and linked with libwm_tensor /
// libwm_hip.  Built by oracle/Makefile into oracle/_ref/run_ref_loss; run on
// the GPU by tests/test_gpu_ref_suites.py.
#include "test_framework.h"

TestSuite* create_loss_tests();

int main() {
    TestRunner runner;
    runner.add_suite(create_loss_tests());
    return runner.run_all();
}
