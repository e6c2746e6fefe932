# burgers1d(loss, u, un, nu, dt, dx, tend, n, nsteps)
#
# Explicit time stepping of the 1-D viscous Burgers equation on n periodic cells,
# central differences for u u_x and u_xx, then the squared-norm loss of the final
# state.  The time loop is a counted loop with a guard (the GPU form of a
# `while tc < tend`): at most nsteps steps, each run only while tc < tend.
#
# loss: length-1 output array, accumulated in place
# u: state of length n, advanced in place
# un: scratch state of length n, overwritten
# nu: viscosity
# dt: time step
# dx: cell size
# tend: final time; a step runs while the elapsed time is below it
# n: number of cells
# nsteps: largest number of steps
function burgers1d(loss, u, un, nu, dt, dx, tend, n, nsteps)
    # coefficients of the advective and diffusive terms
    cadv = 0.5 * dt / dx
    cdif = nu * dt / (dx * dx)
    tc = 0.0
    # the time loop carries the state from step to step (rule 1)
    for i_t = 1:nsteps
        if tc < tend
            # one step, one cell per iteration, periodic neighbours
            for i_x = 1:n
                im = mod(i_x - 2, n) + 1
                ip = mod(i_x, n) + 1
                uc = u[i_x]
                un[i_x] = uc - cadv * uc * (u[ip] - u[im]) + cdif * (u[ip] - 2.0 * uc + u[im])
            end
            # the new state becomes the current one
            for i_x2 = 1:n
                u[i_x2] = un[i_x2]
            end
            tc = tc + dt
        end
    end
    # squared norm of the final state
    for i_k = 1:n
        loss[1] = loss[1] + u[i_k] ^ 2
    end
    return nothing
end
