// A few helper threads that finish sampled rows beside the calling thread.
//
// run(parts, job) calls job(0) on the caller and job(1) .. job(parts - 1) on
// helpers, and returns when every part is done, rethrowing the first
// exception a part raised.  Helpers are started by the first run that asks
// for them and wait on a condition variable between runs; they are joined
// when the crew is destroyed.  One crew serves one caller at a time.
#pragma once

#include <condition_variable>
#include <exception>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

namespace qwen3::generation::detail
{
    class RowCrew final
    {
    public:
        static constexpr int kMaxParts = 4;

        RowCrew() = default;
        RowCrew(const RowCrew &) = delete;
        RowCrew &operator=(const RowCrew &) = delete;

        ~RowCrew()
        {
            {
                std::lock_guard<std::mutex> lock(mutex_);
                quit_ = true;
            }
            go_.notify_all();
            for (std::thread &t : threads_)
                t.join();
        }

        void run(int parts, const std::function<void(int)> &job)
        {
            if (parts > kMaxParts)
                parts = kMaxParts;
            if (parts <= 1)
            {
                job(0);
                return;
            }
            {
                std::unique_lock<std::mutex> lock(mutex_);
                while (static_cast<int>(threads_.size()) < parts - 1)
                {
                    const int part = static_cast<int>(threads_.size()) + 1;
                    threads_.emplace_back([this, part] { helper(part); });
                }
                job_ = &job;
                parts_ = parts;
                pending_ = parts - 1;
                error_ = nullptr;
                ++generation_;
            }
            go_.notify_all();
            std::exception_ptr mine;
            try
            {
                job(0);
            }
            catch (...)
            {
                mine = std::current_exception();
            }
            std::unique_lock<std::mutex> lock(mutex_);
            done_.wait(lock, [this] { return pending_ == 0; });
            job_ = nullptr;
            if (mine)
                std::rethrow_exception(mine);
            if (error_)
                std::rethrow_exception(error_);
        }

    private:
        void helper(int part)
        {
            unsigned long seen = 0;
            std::unique_lock<std::mutex> lock(mutex_);
            for (;;)
            {
                go_.wait(lock, [&] { return quit_ || generation_ != seen; });
                if (quit_)
                    return;
                seen = generation_;
                if (part >= parts_)
                    continue;
                const std::function<void(int)> *job = job_;
                lock.unlock();
                std::exception_ptr failed;
                try
                {
                    (*job)(part);
                }
                catch (...)
                {
                    failed = std::current_exception();
                }
                lock.lock();
                if (failed && !error_)
                    error_ = failed;
                if (--pending_ == 0)
                    done_.notify_one();
            }
        }

        std::mutex mutex_;
        std::condition_variable go_, done_;
        std::vector<std::thread> threads_;
        const std::function<void(int)> *job_ = nullptr;
        unsigned long generation_ = 0;
        int parts_ = 0;
        int pending_ = 0;
        bool quit_ = false;
        std::exception_ptr error_;
    };
} // namespace qwen3::generation::detail
