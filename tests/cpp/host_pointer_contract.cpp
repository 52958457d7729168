// The host-pointer contract of the drop-in Tensor storage (wm::DeviceVector),
// exercised through the reference's class API: a pointer or iterator from a
// non-const data()/begin()/operator[] is valid until the next device
// operation that reads or writes the vector; writes through it before that
// operation are seen by it, writes after it are not (take the pointer again).
// Prints one line per check and exits non-zero on the first failure.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "amp.h"
#include "optimizer.h"
#include "tensor.h"

static int fails = 0;
static void check(bool ok, const char* what) {
    std::printf("%s %s\n", ok ? "OK  " : "FAIL", what);
    if (!ok) ++fails;
}

int main() {
    auto t = Tensor::create(std::vector<float>(1024, 1.0f), {1024}, false);
    // 1. writes through a fresh pointer reach the next op
    float* p = t->data.data();
    p[0] = 5.0f;
    auto y = t->mul(2.0f);
    check(y->data[0] == 10.0f, "write through data() before an op is seen by the op");
    // 2. the same pointer kept across that op: later writes are not seen
    p[1] = 7.0f;
    auto z = t->mul(2.0f);
    check(z->data[1] == 2.0f, "write through a pointer kept across an op is not seen (documented)");
    // 3. taking the pointer again after the op makes writes visible
    t->data.data()[1] = 7.0f;
    auto z2 = t->mul(2.0f);
    check(z2->data[1] == 14.0f, "write through data() taken again after the op is seen");
    // 4. iterators follow the same rule
    for (auto it = t->data.begin(); it != t->data.end(); ++it) *it = 3.0f;
    auto w = t->mul(2.0f);
    check(w->data[1023] == 6.0f, "writes through begin()/end() before an op are seen");
    // 5. a device update (an optimizer step) is seen by a host read taken after it
    auto prm = Tensor::create(std::vector<float>(256, 1.0f), {256}, true);
    prm->grad = std::vector<float>(256, 0.5f);
    const float before = prm->data[0];
    SGD opt({prm}, 0.1f);
    opt.step();
    check(before == 1.0f && prm->data[0] == 0.95f, "a host read after a device update sees the update");
    // 6. const access never marks the device copy stale: reading does not force a re-upload
    const auto& cd = prm->data;
    float s = 0.0f;
    for (float v : cd) s += v;
    auto u = prm->mul(1.0f);
    check(s > 243.19f && s < 243.21f && u->data[5] == 0.95f, "const reads leave the device copy current");
    // 7. HalfVector(n) holds n zeros, as std::vector<uint16_t>(n) does, on the host and on the device
    wm::HalfVector hv(1001);
    bool zeros = hv.size() == 1001;
    for (uint16_t v : hv) zeros = zeros && v == 0;
    auto hf = HalfTensor(Tensor::create(std::vector<float>(8, 2.0f), {8}, false));
    hf.data = wm::HalfVector(8);
    auto back = hf.to_float();
    for (float v : back->data) zeros = zeros && v == 0.0f;
    check(zeros, "HalfVector(n) is n zeros (host reads and a device conversion)");
    std::printf("%s\n", fails ? "CONTRACT BROKEN" : "CONTRACT HOLDS");
    return fails ? 1 : 0;
}
