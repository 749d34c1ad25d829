// The engine: one batch per step through the scheduler and the model runner.
// The contract (the interface of src/inference_engine.h:14-78, pinned by the
// engine tests in tests/cpp): a step schedules a batch, builds its model
// batch, opens the state's transaction, has the runner execute it, checks that
// the runner returned one sample per sampling item and completes the batch.
// Any failure after scheduling aborts the reservation, so the same work is
// scheduled again; the step then reports the failure, or, if the abort itself
// fails, batch_abort_failed with the original failure in its detail.
#include "inference_engine.h"

#include <chrono>

namespace chibillm {

namespace {

using clock = std::chrono::steady_clock;

double
seconds_since(clock::time_point start) noexcept
{
    return std::chrono::duration<double>(clock::now() - start).count();
}

} // namespace

result<inference_engine, inference_engine_error>
inference_engine::make(scheduler_config config, model_runner& runner)
{
    auto state = runner.make_state(config);
    if (!state)
        return fail(inference_engine_errc::scheduler_creation_failed, state.error(),
                    "create model state");
    auto made = scheduler::make(config, runner.info().eos_token, std::move(*state));
    if (!made)
        return fail(inference_engine_errc::scheduler_creation_failed, made.error());
    return inference_engine(std::move(*made), runner);
}

result<void, inference_engine_error>
inference_engine::add(seq sequence)
{
    if (auto added = scheduler_.add(std::move(sequence)); !added)
        return fail(inference_engine_errc::sequence_add_failed, added.error());
    return {};
}

result<admission_result, inference_engine_error>
inference_engine::try_add(seq& sequence)
{
    auto outcome = scheduler_.try_add(sequence);
    if (!outcome)
        return fail(inference_engine_errc::sequence_add_failed, outcome.error());
    return *outcome;
}

result<std::vector<sequence_update>, inference_engine_error>
inference_engine::step()
{
    const auto start = clock::now();
    auto scheduled = scheduler_.schedule();
    times_.schedule_s += seconds_since(start);
    if (!scheduled)
        return fail(inference_engine_errc::scheduling_failed, scheduled.error());
    ++times_.steps;
    auto outcome = run(*scheduled);
    if (!outcome)
        return abandon(*scheduled, std::move(outcome.error()));
    return std::move(*outcome);
}

// The reserved batch from model batch to completion; the caller aborts the
// reservation when this fails.
result<std::vector<sequence_update>, inference_engine_error>
inference_engine::run(const scheduled_batch& scheduled)
{
    using errc = inference_engine_errc;
    auto start = clock::now();
    auto batch = build_model_batch(scheduled, scheduler_);
    times_.build_s += seconds_since(start);
    if (!batch)
        return fail(inference_engine_error { errc::model_batch_build_failed,
                                             describe_error(batch.error()) });
    if (auto begun = scheduler_.begin_execution(*batch); !begun)
        return fail(inference_engine_error { errc::model_execution_failed,
                                             "begin batch: " + describe_error(begun.error()) });
    start = clock::now();
    auto samples = runner_->execute(*batch, scheduler_.state());
    times_.execute_s += seconds_since(start);
    if (!samples)
        return fail(inference_engine_error { errc::model_execution_failed,
                                             describe_error(samples.error()) });
    const std::size_t wanted = batch->sample_count();
    if (samples->size() != wanted)
        return fail(inference_engine_error {
            errc::runner_result_count_mismatch,
            "expected " + std::to_string(wanted) + " samples, received "
                + std::to_string(samples->size()) });
    start = clock::now();
    auto updates = scheduler_.complete(scheduled.id, *samples);
    times_.complete_s += seconds_since(start);
    if (!updates)
        return fail(inference_engine_error { errc::batch_completion_failed,
                                             describe_error(updates.error()) });
    return std::move(*updates);
}

failure<inference_engine_error>
inference_engine::abandon(const scheduled_batch& batch, inference_engine_error cause)
{
    if (auto aborted = scheduler_.abort(batch.id); !aborted)
        return fail(inference_engine_error { inference_engine_errc::batch_abort_failed,
                                             describe_error(aborted.error())
                                                 + "; original failure: "
                                                 + describe_error(cause) });
    return fail(std::move(cause));
}

result<void, inference_engine_error>
inference_engine::cancel(seq_id id)
{
    if (auto cancelled = scheduler_.cancel(id); !cancelled)
        return fail(inference_engine_errc::sequence_cancel_failed, cancelled.error());
    return {};
}

result<void, inference_engine_error>
inference_engine::remove(seq_id id)
{
    if (auto removed = scheduler_.remove(id); !removed)
        return fail(inference_engine_errc::sequence_remove_failed, removed.error());
    return {};
}

} // namespace chibillm
