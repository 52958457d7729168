// ref_layers_main.cpp -- TEST INFRASTRUCTURE ONLY.
//
// Runner for the reference's own layer suite (tests/test_layers.cpp in the
// reference), compiled where it lies against this build's drop-in Tensor and
// modules (whitematter_amd/core/tensor.h and layer.h, force-included so that
// they stand in for the reference's headers) and linked with libwm_tensor /
// libwm_hip.  Built by oracle/Makefile into oracle/_ref/run_ref_layers; run
// on the GPU by tests/test_gpu_ref_suites.py.
#include "test_framework.h"

TestSuite* create_layer_tests();

int main() {
    TestRunner runner;
    runner.add_suite(create_layer_tests());
    return runner.run_all();
}
