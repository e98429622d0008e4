// TEST DRIVER (checker side): runs the reference-side adapter
// (integration/hip_backend.cpp) on the GPU through the reference's own
// interfaces -- gpu::Device/Queue, kernels::prepare/PreparedOperation,
// DeviceCategorical, DeviceSequence, DeviceInjection, DeviceDirection and
// DeviceIntervention -- and checks every result against the CPU oracle
// (oracle/liboracle.so).  Built by integration/Makefile against the
// reference headers (with the reference's kernels/operations.cpp and
// tensors/tensor.cpp for validate_operation and the layout helpers); run by
// tests/test_gpu_adapter.py.  Prints "ok <check>" per check and exits 1 on
// the first mismatch.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <random>
#include <stdexcept>
#include <stop_token>
#include <string>
#include <vector>

#include "gpu/device.h"
#include "inference/cache/contiguous.h"
#include "inference/decoding/device.h"
#include "inference/injection/device.h"
#include "inference/observations.h"
#include "inference/sampling/device.h"
#include "inference/steering/device.h"
#include "kernels/operations.h"
#include "tensors/tensor.h"

extern "C" {
#include "oracle.h"
}

namespace dolittle::gpu::hip {
std::unique_ptr<Device> open_device(int ordinal);
}

using namespace dolittle;
using tensors::ElementType;

namespace {

[[noreturn]] void fail(const std::string& what) {
  std::fprintf(stdout, "FAIL %s\n", what.c_str());
  std::fflush(stdout);
  std::exit(1);
}
void ok(const std::string& what) {
  std::fprintf(stdout, "ok %s\n", what.c_str());
  std::fflush(stdout);
}

std::vector<std::uint16_t> random_bf16(std::size_t n, std::uint64_t seed, float scale) {
  std::mt19937_64 rng(seed);
  std::normal_distribution<float> normal(0.0f, scale);
  std::vector<std::uint16_t> v(n);
  for (auto& x : v) x = or_bf16_from_f32(normal(rng));
  return v;
}

// Device buffers filled from and read back to host vectors through staging
// buffers and the adapter's Queue.
struct Harness {
  std::unique_ptr<gpu::Device> device = gpu::hip::open_device(0);
  gpu::Queue queue = device->create_queue();

  template <class T>
  gpu::DeviceBuffer upload(const std::vector<T>& host, std::size_t extra = 0) {
    const std::size_t bytes = host.size() * sizeof(T) + extra;
    auto buffer = device->allocate({bytes, 256});
    auto staging = device->allocate_staging({bytes, 64});
    std::memset(staging.bytes().data(), 0, bytes);
    std::memcpy(staging.bytes().data(), host.data(), host.size() * sizeof(T));
    queue.upload({&buffer, 0, bytes}, {&staging, 0, bytes});
    queue.drain();
    return buffer;
  }
  template <class T>
  std::vector<T> download(gpu::ConstDeviceRegion region) {
    auto staging = device->allocate_staging({region.bytes, 64});
    queue.download({&staging, 0, region.bytes}, region);
    queue.drain();
    std::vector<T> out(region.bytes / sizeof(T));
    std::memcpy(out.data(), staging.bytes().data(), region.bytes);
    return out;
  }
  template <class T>
  std::vector<T> download(const gpu::DeviceBuffer& buffer) {
    return download<T>(gpu::ConstDeviceRegion{&buffer, 0, buffer.size_bytes()});
  }
};

tensors::Layout layout(ElementType t, std::vector<std::size_t> shape) {
  return tensors::contiguous_layout(t, shape);
}

constexpr tensors::ComputationMode kMode{ElementType::bfloat16, ElementType::float32};

template <class T>
void expect_equal(const std::vector<T>& got, const std::vector<T>& want, const std::string& what) {
  if (got.size() < want.size()) fail(what + ": short result");
  for (std::size_t i = 0; i < want.size(); ++i)
    if (got[i] != want[i]) fail(what + ": element " + std::to_string(i) + " differs");
  ok(what);
}

// Runs one prepared operation over the given bound buffers.
void run(Harness& h, const kernels::Operation& op, const std::vector<tensors::Layout>& layouts,
         std::vector<kernels::BufferBinding> bindings, kernels::RowPolicy rows = {},
         const kernels::ExecutionExtent* extent = nullptr, const inference::cache::ContiguousLayerView* view = nullptr) {
  auto prepared = kernels::prepare(*h.device, op, layouts, kMode, rows);
  const auto need = prepared.workspace();
  std::unique_ptr<gpu::DeviceBuffer> constants;
  gpu::DeviceRegion workspace{nullptr, 0, 0};
  if (need.bytes) {
    constants = std::make_unique<gpu::DeviceBuffer>(h.device->allocate({need.bytes, need.alignment}));
    workspace = {constants.get(), 0, need.bytes};
    prepared.initialize(h.queue, workspace);
  }
  prepared.submit(h.queue, bindings, workspace, extent, view);
  h.queue.drain();
}

kernels::BufferBinding in(std::size_t id, const gpu::DeviceBuffer& b) {
  return {{id}, static_cast<const gpu::DeviceBuffer*>(&b), 0, b.size_bytes()};
}
kernels::BufferBinding out(std::size_t id, gpu::DeviceBuffer& b) { return {{id}, &b, 0, b.size_bytes()}; }

void transfers_and_sampler(Harness& h) {
  const auto values = random_bf16(4096, 1, 1.0f);
  auto a = h.upload(values);
  auto b = h.device->allocate({a.size_bytes(), 256});
  h.queue.copy({&b, 0, b.size_bytes()}, {&a, 0, a.size_bytes()});
  expect_equal(h.download<std::uint16_t>(b), values, "queue upload, copy and download");

  // DeviceCategorical's result words are borrowed regions; the reference
  // downloads the region submit() returns (executor.cpp:1021).
  const std::size_t vocabulary = 513;
  std::vector<std::uint16_t> logits(vocabulary);
  for (std::size_t i = 0; i < vocabulary; ++i) logits[i] = or_bf16_from_f32(static_cast<float>(i % 97) / 8.0f - 6.0f);
  auto row = h.upload(logits);
  inference::sampling::DeviceCategorical sampler(*h.device, h.queue, vocabulary, ElementType::bfloat16,
                                                 inference::sampling::DeviceCategorical::required_bytes(vocabulary));
  sampler.start({inference::sampling::SelectionMode::greedy, 1.0, 0, 1.0}, 5, {});
  const auto result = sampler.submit_next({&row, 0, row.size_bytes()});
  const auto words = h.download<std::uint32_t>(result);
  std::uint32_t want = 0;
  if (orc_greedy_bf16(logits.data(), vocabulary, &want) != 0) fail("oracle greedy");
  if (words.size() != 2 || words[0] != want || words[1] != 0) fail("sampler result region download");
  ok("DeviceCategorical::submit_next result region downloaded");
  const auto token = h.download<std::uint32_t>(sampler.current_token());
  if (token[0] != want) fail("sampler current token region");
  ok("DeviceCategorical::current_token region downloaded");
}

void operations(Harness& h) {
  using namespace kernels;
  {  // Projection [5, 256] x [64, 256]^T
    const auto x = random_bf16(5 * 256, 2, 1.0f), w = random_bf16(64 * 256, 3, 0.05f);
    auto bx = h.upload(x), bw = h.upload(w);
    auto by = h.device->allocate({5 * 64 * 2, 256});
    run(h, Projection{{0}, {1}, {2}},
        {layout(ElementType::bfloat16, {5, 256}), layout(ElementType::bfloat16, {64, 256}),
         layout(ElementType::bfloat16, {5, 64})},
        {in(0, bx), in(1, bw), out(2, by)});
    std::vector<std::uint16_t> want(5 * 64);
    orc_projection(x.data(), w.data(), want.data(), 5, 256, 64);
    expect_equal(h.download<std::uint16_t>(by), want, "prepared Projection");
  }
  {  // RmsNorm [5, 256]
    const auto x = random_bf16(5 * 256, 4, 2.0f), g = random_bf16(256, 5, 1.0f);
    auto bx = h.upload(x), bg = h.upload(g);
    auto by = h.device->allocate({5 * 256 * 2, 256});
    run(h, RmsNorm{{0}, {1}, {2}, 1e-6f},
        {layout(ElementType::bfloat16, {5, 256}), layout(ElementType::bfloat16, {256}),
         layout(ElementType::bfloat16, {5, 256})},
        {in(0, bx), in(1, bg), out(2, by)});
    std::vector<std::uint16_t> want(5 * 256);
    orc_rms_norm(x.data(), g.data(), want.data(), 5, 256, 1e-6f);
    expect_equal(h.download<std::uint16_t>(by), want, "prepared RmsNorm");
  }
  {  // Rotary [3, 4, 128] at position 7
    const auto x = random_bf16(3 * 4 * 128, 6, 1.0f);
    auto bx = h.upload(x);
    auto by = h.device->allocate({x.size() * 2, 256});
    run(h, Rotary{{0}, {1}, 7, 1e6},
        {layout(ElementType::bfloat16, {3, 4, 128}), layout(ElementType::bfloat16, {3, 4, 128})},
        {in(0, bx), out(1, by)});
    std::vector<std::uint16_t> want(x.size());
    orc_rotary(x.data(), want.data(), 3, 4, 128, 7, 1e6);
    expect_equal(h.download<std::uint16_t>(by), want, "prepared Rotary");
  }
  {  // CausalAttention, static: Q [6, 4, 128], K/V [6, 2, 128]
    const auto q = random_bf16(6 * 4 * 128, 7, 1.0f), k = random_bf16(6 * 2 * 128, 8, 1.0f),
               v = random_bf16(6 * 2 * 128, 9, 1.0f);
    auto bq = h.upload(q), bk = h.upload(k), bv = h.upload(v);
    auto by = h.device->allocate({q.size() * 2, 256});
    run(h, CausalAttention{{0}, {1}, {2}, {3}},
        {layout(ElementType::bfloat16, {6, 4, 128}), layout(ElementType::bfloat16, {6, 2, 128}),
         layout(ElementType::bfloat16, {6, 2, 128}), layout(ElementType::bfloat16, {6, 4, 128})},
        {in(0, bq), in(1, bk), in(2, bv), out(3, by)});
    std::vector<std::uint16_t> want(q.size());
    orc_attention(q.data(), k.data(), v.data(), want.data(), 6, 4, 2, 128, 0, 2 * 128, 128);
    expect_equal(h.download<std::uint16_t>(by), want, "prepared CausalAttention (full forward)");
  }
  {  // CausalAttention, dynamic: 2 active rows of 4 at position 9 over a
     // 16-row cache view (the executor's incremental form).
    const std::size_t cap = 16, first = 9, rows = 2, max_rows = 4;
    const auto q = random_bf16(max_rows * 4 * 128, 10, 1.0f);
    const auto k = random_bf16(cap * 2 * 128, 11, 1.0f), v = random_bf16(cap * 2 * 128, 12, 1.0f);
    auto bq = h.upload(q), bk = h.upload(k), bv = h.upload(v);
    auto by = h.device->allocate({q.size() * 2, 256});
    auto kq = h.upload(std::vector<std::uint16_t>(max_rows * 2 * 128)), vq = h.upload(std::vector<std::uint16_t>(max_rows * 2 * 128));
    const inference::cache::ContiguousLayerView view{
        {&bk, 0, bk.size_bytes()}, {&bv, 0, bv.size_bytes()}, cap, {2, 128}};
    const ExecutionExtent extent{first, rows, nullptr, 0};
    run(h, CausalAttention{{0}, {1}, {2}, {3}},
        {layout(ElementType::bfloat16, {max_rows, 4, 128}), layout(ElementType::bfloat16, {max_rows, 2, 128}),
         layout(ElementType::bfloat16, {max_rows, 2, 128}), layout(ElementType::bfloat16, {max_rows, 4, 128})},
        {in(0, bq), in(1, kq), in(2, vq), out(3, by)}, RowPolicy{max_rows, false}, &extent, &view);
    std::vector<std::uint16_t> want(rows * 4 * 128);
    orc_attention(q.data(), k.data(), v.data(), want.data(), rows, 4, 2, 128, first, 2 * 128, 128);
    expect_equal(h.download<std::uint16_t>(by), want, "prepared CausalAttention (cache view, dynamic rows)");
  }
  {  // Embedding, Add, SiluMultiply
    const std::vector<std::uint32_t> ids = {3, 0, 31, 7};
    const auto table = random_bf16(32 * 64, 13, 1.0f);
    auto bt = h.upload(ids), bw = h.upload(table);
    auto by = h.device->allocate({4 * 64 * 2, 256});
    run(h, Embedding{{0}, {1}, {2}},
        {layout(ElementType::uint32, {4}), layout(ElementType::bfloat16, {32, 64}),
         layout(ElementType::bfloat16, {4, 64})},
        {in(0, bt), in(1, bw), out(2, by)});
    std::vector<std::uint16_t> want(4 * 64);
    orc_embedding(ids.data(), table.data(), want.data(), 4, 64);
    expect_equal(h.download<std::uint16_t>(by), want, "prepared Embedding");

    const auto a = random_bf16(1000, 14, 3.0f), b = random_bf16(1000, 15, 3.0f);
    auto ba = h.upload(a), bb = h.upload(b);
    auto bs = h.device->allocate({2000, 256}), bm = h.device->allocate({2000, 256});
    const auto l = layout(ElementType::bfloat16, {10, 100});
    run(h, Add{{0}, {1}, {2}}, {l, l, l}, {in(0, ba), in(1, bb), out(2, bs)});
    run(h, SiluMultiply{{0}, {1}, {2}}, {l, l, l}, {in(0, ba), in(1, bb), out(2, bm)});
    std::vector<std::uint16_t> want_add(1000), want_silu(1000);
    orc_add(a.data(), b.data(), want_add.data(), 1000);
    orc_silu_multiply(a.data(), b.data(), want_silu.data(), 1000);
    expect_equal(h.download<std::uint16_t>(bs), want_add, "prepared Add");
    expect_equal(h.download<std::uint16_t>(bm), want_silu, "prepared SiluMultiply");
  }
  {  // GatherRows {0, 2, 3} of [5, 64], and the last-row policy at 3 of 5 rows
    const auto x = random_bf16(5 * 64, 16, 1.0f);
    auto bx = h.upload(x);
    auto by = h.device->allocate({3 * 64 * 2, 256});
    run(h, GatherRows{{0}, {1}, {0, 2, 3}},
        {layout(ElementType::bfloat16, {5, 64}), layout(ElementType::bfloat16, {3, 64})},
        {in(0, bx), out(1, by)});
    std::vector<std::uint16_t> want;
    for (int r : {0, 2, 3}) want.insert(want.end(), x.begin() + r * 64, x.begin() + (r + 1) * 64);
    expect_equal(h.download<std::uint16_t>(by), want, "prepared GatherRows");
    auto bl = h.device->allocate({64 * 2, 256});
    const ExecutionExtent extent{0, 3, nullptr, 0};
    run(h, GatherRows{{0}, {1}, {4}},
        {layout(ElementType::bfloat16, {5, 64}), layout(ElementType::bfloat16, {1, 64})},
        {in(0, bx), out(1, bl)}, RowPolicy{5, true}, &extent);
    expect_equal(h.download<std::uint16_t>(bl), std::vector<std::uint16_t>(x.begin() + 2 * 64, x.begin() + 3 * 64),
                 "prepared GatherRows (last active row)");
  }
}

// A toy recipe recorded into a DeviceSequence the way the executor records
// the Qwen3 one (executor.cpp:1595-1657): Embedding of the body's token rows
// (captured), then the last row's logits Projection and the device sampler.
// Greedy makes it a Markov chain the oracle follows:
// next = argmax(W E[token]).
struct ToySequence {
  static constexpr std::size_t V = 256, D = 128;
  std::vector<std::uint16_t> table = random_bf16(V * D, 21, 1.0f), head = random_bf16(V * D, 22, 0.2f);

  std::uint32_t next(std::uint32_t token) const {
    std::vector<std::uint16_t> logits(V);
    orc_projection(table.data() + token * D, head.data(), logits.data(), 1, D, V);
    std::uint32_t id = 0;
    if (orc_greedy_bf16(logits.data(), V, &id) != 0) fail("oracle greedy");
    return id;
  }

  struct Outcome {
    std::vector<inference::DeviceSequence::Event> events;
    std::vector<std::uint16_t> captures;
  };

  Outcome run(Harness& h, const std::vector<std::uint32_t>& prompt, std::size_t generated, std::size_t chunk,
              std::vector<std::uint32_t> stops, bool cancel_first) {
    using namespace kernels;
    using inference::DeviceSequence;
    const std::size_t P = prompt.size(), capacity = P + generated;
    auto tokens = h.device->allocate({chunk * 4, 256});
    auto hidden = h.device->allocate({chunk * D * 2, 256});
    auto last = h.device->allocate({D * 2, 256});
    auto logits = h.device->allocate({V * 2, 256});
    auto arena = h.device->allocate({capacity * D * 2, 256});
    auto ids = h.upload(prompt);
    auto bt = h.upload(table), bh = h.upload(head);
    inference::sampling::DeviceCategorical sampler(*h.device, h.queue, V, ElementType::bfloat16,
                                                   inference::sampling::DeviceCategorical::required_bytes(V));
    sampler.start({inference::sampling::SelectionMode::greedy, 1.0, 0, 1.0}, 1, stops);
    const std::vector<tensors::Layout> layouts = {
        layout(ElementType::uint32, {chunk}), layout(ElementType::bfloat16, {V, D}),
        layout(ElementType::bfloat16, {chunk, D}), layout(ElementType::bfloat16, {1, D}),
        layout(ElementType::bfloat16, {1, V})};
    auto embed = prepare(*h.device, Embedding{{0}, {1}, {2}}, layouts, kMode, {chunk, false});
    auto gather = prepare(*h.device, GatherRows{{2}, {3}, {chunk - 1}}, layouts, kMode, {chunk, true});
    auto project = prepare(*h.device, Projection{{3}, {1}, {4}}, layouts, kMode, {});
    const std::vector<BufferBinding> embed_bind = {in(0, tokens), in(1, bt), out(2, hidden)};
    const std::vector<BufferBinding> gather_bind = {in(2, hidden), out(3, last)};
    const std::vector<BufferBinding> project_bind = {in(3, last), in(1, bh), out(4, logits)};

    DeviceSequence sequence(*h.device, h.queue, {P, generated, chunk, false});
    const auto position = sequence.position();
    const gpu::DeviceRegion none{nullptr, 0, 0};
    auto forward = [&](std::size_t rows) {
      const ExecutionExtent extent{0, rows, &position, capacity};
      embed.submit(h.queue, embed_bind, none, &extent);
      sequence.capture({&hidden, 0, rows * D * 2}, {&arena, 0, arena.size_bytes()}, D * 2, rows);
    };
    auto select = [&](std::size_t rows) {
      const ExecutionExtent extent{0, rows, &position, capacity};
      gather.submit(h.queue, gather_bind, none, &extent);
      project.submit(h.queue, project_bind, none);
      (void)sampler.submit_next({&logits, 0, logits.size_bytes()});
    };
    sequence.begin(sampler.result_storage(), sampler.terminal_state(), {&tokens, 0, tokens.size_bytes()},
                   {&ids, 0, ids.size_bytes()});
    sequence.begin_stage(DeviceSequence::Stage::prefill);
    forward(chunk);
    sequence.end_stage();
    sequence.begin_stage(DeviceSequence::Stage::tail);
    if (P % chunk) forward(P % chunk);
    sequence.end_stage();
    sequence.begin_stage(DeviceSequence::Stage::first_selection);
    select(P % chunk ? P % chunk : chunk);
    sequence.end_stage();
    sequence.begin_stage(DeviceSequence::Stage::decode);
    forward(1);
    sequence.begin_selection();
    select(1);
    sequence.end_stage();
    sequence.complete();
    if (cancel_first) sequence.request_stop();
    sequence.start();
    Outcome outcome;
    std::stop_source source;
    for (std::size_t i = 0;; ++i) {
      outcome.events.push_back(sequence.collect(i, source.get_token()));
      if (outcome.events.back().kind == DeviceSequence::Kind::terminal) break;
    }
    sequence.drain();
    outcome.captures = h.download<std::uint16_t>(arena);
    return outcome;
  }
};

void sequence(Harness& h) {
  using Kind = inference::DeviceSequence::Kind;
  ToySequence toy;
  const std::vector<std::uint32_t> prompt = {5, 17, 200, 3, 99, 41, 7};
  const std::size_t P = prompt.size(), chunk = 3;
  // The oracle's stream.
  std::vector<std::uint32_t> stream = prompt;
  for (int i = 0; i < 6; ++i) stream.push_back(toy.next(stream.back()));

  auto expect = [&](const ToySequence::Outcome& o, std::size_t generated, std::uint32_t reason,
                    const std::string& what, std::size_t P) {
    std::size_t consumed = 0, selected = 0;
    for (std::size_t i = 0; i + 1 < o.events.size(); ++i) {
      const auto& e = o.events[i];
      if (e.kind == Kind::consumed) {
        if (e.position != consumed) fail(what + ": consumed event position");
        consumed += e.count;
      } else if (e.kind == Kind::selected) {
        if (e.position != P + selected || e.token != stream[P + selected]) fail(what + ": selected token");
        ++selected;
      } else {
        fail(what + ": unexpected event kind");
      }
    }
    const auto& t = o.events.back();
    if (selected != generated || t.count != generated || t.status != reason || t.position != consumed)
      fail(what + ": terminal event");
    for (std::size_t pos = 0; pos < consumed; ++pos)
      for (std::size_t f = 0; f < ToySequence::D; ++f)
        if (o.captures[pos * ToySequence::D + f] != toy.table[stream[pos] * ToySequence::D + f])
          fail(what + ": capture row " + std::to_string(pos));
    ok(what);
  };

  // Limit: 7-id prompt in chunks of 3 (two chunks and a remainder), five
  // tokens, every selection consumed (terminal at position 12).
  auto limit = toy.run(h, prompt, 5, chunk, {}, false);
  if (limit.events.size() != 3 + 1 + 2 * 4 + 1 + 1) fail("limit: event count");
  expect(limit, 5, 0, "DeviceSequence limit: events, tokens and captures against the oracle", P);
  // EOS: the second generated token is a stop id (the stream may repeat
  // tokens, so the stop is its first occurrence); it is still consumed.
  const std::uint32_t stop = stream[P + 1];
  std::size_t stop_at = 0;
  while (stream[P + stop_at] != stop) ++stop_at;
  auto eos = toy.run(h, prompt, 5, chunk, {stop}, false);
  expect(eos, stop_at + 1, 1, "DeviceSequence eos: the stop token is selected and consumed", P);
  // Cancelled before start: nothing runs.
  auto cancelled = toy.run(h, prompt, 5, chunk, {}, true);
  if (cancelled.events.size() != 1) fail("cancel: events");
  expect(cancelled, 0, 2, "DeviceSequence cancelled before start", P);
  // Whole-chunk prompt (no remainder) and chunk 1.
  auto exact = toy.run(h, {5, 17, 200, 3, 99, 41}, 3, 3, {}, false);
  stream = {5, 17, 200, 3, 99, 41};
  for (int i = 0; i < 3; ++i) stream.push_back(toy.next(stream.back()));
  expect(exact, 3, 0, "DeviceSequence prompt of whole chunks", 6);
}

void nla(Harness& h) {
  const std::size_t width = 4096;
  const auto source = random_bf16(width, 31, 1.0f);
  auto bs = h.upload(source);
  inference::DeviceInjection injection(*h.device, h.queue, {&bs, 0, bs.size_bytes()}, ElementType::bfloat16,
                                       ElementType::bfloat16, width, 150.0f);
  injection.submit();
  std::vector<std::uint16_t> want(width);
  float norm = 0.0f;
  const std::uint32_t status = orc_inject(source.data(), 1, want.data(), 1, width, 150.0f, &norm);
  const auto got = h.download<std::uint16_t>(injection.output());
  const auto got_status = h.download<std::uint32_t>(injection.status());
  const auto got_norm = h.download<float>(injection.norm());
  if (got_status[0] != status || std::memcmp(&got_norm[0], &norm, 4) != 0) fail("DeviceInjection status/norm");
  expect_equal(got, want, "DeviceInjection output, status and norm");

  auto original = std::make_shared<gpu::DeviceBuffer>(h.upload(random_bf16(width, 32, 1.0f)));
  const auto edited_host = random_bf16(width, 33, 1.0f);
  auto edited = std::make_shared<gpu::DeviceBuffer>(h.upload(edited_host));
  const auto original_host = h.download<std::uint16_t>(*original);
  inference::DeviceDirection direction(*h.device, h.queue, {original, 0, width * 2}, {edited, 0, width * 2},
                                       ElementType::bfloat16, width);
  direction.submit();
  const auto capture = direction.finish();
  std::vector<float> want_dir(width);
  if (orc_direction(original_host.data(), edited_host.data(), 1, width, want_dir.data()) != 0) fail("oracle direction");
  expect_equal(h.download<float>(capture.region()), want_dir, "DeviceDirection");

  // One-row intervention at position 11 of a 3-row chunk at position 10.
  const auto residual = random_bf16(3 * width, 34, 2.0f);
  auto br = h.upload(residual);
  auto bp = h.upload(std::vector<std::uint64_t>{10});
  inference::ResidualIntervention input{};
  input.position.value = 11;
  input.direction = capture;
  input.width = width;
  input.strength = 0.5f;
  inference::DeviceIntervention intervention(*h.device, h.queue, input, ElementType::bfloat16);
  intervention.initialize();
  intervention.submit({&br, 0, br.size_bytes()}, {&bp, 0, 8}, 3);
  auto want_res = residual;
  std::uint32_t state[2] = {0, 0};
  (void)orc_intervene(want_res.data(), 1, 3, width, want_dir.data(), 10, 11, 0.5f, state);
  const auto got_status2 = h.download<std::uint32_t>(intervention.status());
  const auto got_count = h.download<std::uint32_t>(intervention.count());
  if (got_status2[0] != state[0] || got_count[0] != state[1] || got_count[0] != 1) fail("DeviceIntervention state");
  expect_equal(h.download<std::uint16_t>(br), want_res, "DeviceIntervention row and state");
}

}  // namespace

int main(int argc, char** argv) {
  const std::string which = argc > 1 ? argv[1] : "all";
  try {
    Harness h;
    if (which == "all" || which == "transfers") transfers_and_sampler(h);
    if (which == "all" || which == "operations") operations(h);
    if (which == "all" || which == "sequence") sequence(h);
    if (which == "all" || which == "nla") nla(h);
  } catch (const std::exception& e) {
    fail(std::string("exception: ") + e.what());
  }
  std::printf("done\n");
  return 0;
}
