// ref_suites_main.cpp -- TEST INFRASTRUCTURE ONLY.
//
// Runner for the reference's own tensor and autograd unit-test suites
// (tests/test_tensor.cpp, tests/test_autograd.cpp in the reference), compiled
// where they lie against this build's drop-in Tensor (whitematter_amd/core/
// tensor.h, force-included so that it stands in for the reference's header)
// and linked with libwm_tensor / libwm_hip.  Built by oracle/Makefile into
// oracle/_ref/run_ref_suites; run on the GPU by tests/test_gpu_ref_suites.py.
#include "test_framework.h"

TestSuite* create_tensor_tests();
TestSuite* create_autograd_tests();

int main() {
    TestRunner runner;
    runner.add_suite(create_tensor_tests());
    runner.add_suite(create_autograd_tests());
    return runner.run_all();
}
